"""lightning_core.api -- the integrated conv -> attention entry points.

Mirrors the reference's `api` submodule (python/bindings/bind_integrated.cpp:
951-1190): conv_relu_nchw[_into], attention[_into],
conv_attention_torchstrong_nchw[_into] and its eager-vs-graph A/B report.
`execution_mode="graph"` runs the graph-mode entry (one HIP graph per shape
key, 3x3 weights only); as in the reference (:925-942), a graph failure falls
back to the eager result unless LC_GRAPH_MODE_STRICT is set, in which case it
raises with the reference's hint.
"""
from __future__ import annotations

import os
import time

import numpy as np

from . import _core
from . import _native as N

__all__ = ["conv_relu_nchw", "conv_relu_nchw_into", "attention", "attention_into",
           "conv_attention_torchstrong_nchw", "conv_attention_torchstrong_nchw_into",
           "conv_attention_torchstrong_nchw_ab_report", "clear_attention_session_cache",
           "clear_conv_attention_graph_cache"]


def _mode(execution_mode: str):
    if execution_mode not in ("eager", "graph"):
        raise ValueError("unsupported execution mode")


def _graph_strict() -> bool:
    """envFlagEnabled("LC_GRAPH_MODE_STRICT") (bind_integrated.cpp:132-146)."""
    raw = os.environ.get("LC_GRAPH_MODE_STRICT", "")
    return raw[:1].lower() in ("1", "t", "y")


_GRAPH_TAG = "conv2d_nchw3x3->qkv_pack_repeat->attention_forward"


def _graph_failure(status: int, device: str) -> str:
    """throwGraphExecuteFailure (bind_integrated.cpp:240-255)."""
    lib = _core._lib()
    msg = f"graph execute_f32 failed ({_GRAPH_TAG}): {lib.lcGetErrorString(status).decode()}"
    detail = lib.lcGetLastErrorMessage().decode()
    if detail:
        msg += f" [{detail}]"
    if status == N.LC_NOT_SUPPORTED:
        msg += (f" | hint: selected backend is unsupported for this path on device='{device}'; "
                "try execution_mode='eager' or device='cpu'")
    elif status == N.LC_INVALID_VALUE:
        msg += " | hint: check feed shapes/numel and conv->attn dimensions (seq_len * head_dim)"
    else:
        msg += " | hint: retry with execution_mode='eager' and compare using *_ab_report API"
    return msg


def conv_relu_nchw(x, w, bias=None, stride_h=1, stride_w=1, pad_h=0, pad_w=0, device="hip"):
    return _core.conv2d_nchw(x, w, bias, stride_h, stride_w, pad_h, pad_w, device, apply_relu=True)


def conv_relu_nchw_into(x, w, bias, out, stride_h=1, stride_w=1, pad_h=0, pad_w=0, device="hip"):
    res = conv_relu_nchw(x, w, bias, stride_h, stride_w, pad_h, pad_w, device)
    if out.size != res.size:
        raise ValueError("out size mismatch")
    out.reshape(-1)[:] = res.reshape(-1)


def attention(q, k, v, seq_len, head_dim, causal=False, device="hip"):
    return _core.attention_forward(q, k, v, seq_len, head_dim, causal, device)


def attention_into(q, k, v, out, seq_len, head_dim, causal=False, device="hip"):
    res = _core.attention_forward(q, k, v, seq_len, head_dim, causal, device)
    if out.size != res.size:
        raise ValueError("out size mismatch")
    out.reshape(-1)[:] = res


def conv_attention_torchstrong_nchw_into(x, w, bias, out, seq_len, head_dim, stride_h=1, stride_w=1, pad_h=0,
                                         pad_w=0, device="hip", execution_mode="eager"):
    """bind_integrated.cpp:614-730, :1100-1130."""
    _mode(execution_mode)
    x, w = _core._f32(x), _core._f32(w)
    if x.ndim != 4 or w.ndim != 4:
        raise ValueError("x and w must be 4D arrays (NCHW and OIHW)")
    bn, c, h, wd = x.shape
    oc, wc, kh, kw = w.shape
    if c != wc:
        raise ValueError("x channels and w in_channels mismatch")
    if stride_h == 0 or stride_w == 0:
        raise ValueError("stride must be > 0")
    if h + 2 * pad_h < kh or wd + 2 * pad_w < kw:
        raise ValueError("invalid padding/kernel for input size")
    b = None
    if bias is not None:
        b = _core._f32(bias).ravel()
        if b.size != oc:
            raise ValueError("bias shape mismatch")
    _core._require_out(out, seq_len * head_dim)
    lib = _core._lib()
    args = (_core._fp(x), _core._fp(w), _core._fp(b), _core._fp(out), bn, c, h, wd, oc, kh, kw, seq_len, head_dim,
            stride_h, stride_w, pad_h, pad_w, _core._parse_device(device))
    if execution_mode == "graph":
        st = lib.lcConvAttentionTorchstrongNchwGraph(*args)
        if st == N.LC_SUCCESS:
            return
        if _graph_strict():
            raise RuntimeError(_graph_failure(st, device))
        # deterministic fallback contract: the eager result (bind_integrated.cpp:937-941)
    _core._check(lib.lcConvAttentionTorchstrongNchw(*args))


def conv_attention_torchstrong_nchw(x, w, bias, seq_len, head_dim, stride_h=1, stride_w=1, pad_h=0, pad_w=0,
                                    device="hip", execution_mode="eager"):
    """bind_integrated.cpp:1059-1098: returns a flat [seq_len*head_dim] array."""
    out = np.empty(seq_len * head_dim, np.float32)
    conv_attention_torchstrong_nchw_into(x, w, bias, out, seq_len, head_dim, stride_h, stride_w, pad_h, pad_w,
                                         device, execution_mode)
    return out


def conv_attention_torchstrong_nchw_ab_report(x, w, bias, seq_len, head_dim, stride_h=1, stride_w=1, pad_h=0,
                                              pad_w=0, device="hip", warmup=1, repeat=5, atol=1e-4, rtol=1e-4):
    """convAttentionTorchstrongNchwAbReport (bind_integrated.cpp:839-911): times
    eager then graph mode and compares their outputs."""
    if repeat == 0:
        raise ValueError("repeat must be > 0")
    if atol < 0.0 or rtol < 0.0:
        raise ValueError("atol/rtol must be >= 0")
    need = seq_len * head_dim

    def run(mode):
        out = np.empty(need, np.float32)
        for _ in range(warmup):
            conv_attention_torchstrong_nchw_into(x, w, bias, out, seq_len, head_dim, stride_h, stride_w, pad_h,
                                                 pad_w, device, mode)
        t0 = time.perf_counter()
        for _ in range(repeat):
            conv_attention_torchstrong_nchw_into(x, w, bias, out, seq_len, head_dim, stride_h, stride_w, pad_h,
                                                 pad_w, device, mode)
        return (time.perf_counter() - t0) * 1e3 / repeat, out

    eager_ms, eager = run("eager")
    graph_ms, graph = run("graph")
    e64, g64 = eager.astype(np.float64), graph.astype(np.float64)
    diff = np.abs(e64 - g64)
    rel = diff / (np.abs(e64) + 1e-12)
    report = {
        "seq_len": seq_len, "head_dim": head_dim, "warmup": warmup, "repeat": repeat, "device": device,
        "allclose": bool(np.all(diff <= atol + rtol * np.abs(e64))),
        "max_abs_diff": float(diff.max()) if need else 0.0,
        "mean_abs_diff": float(diff.mean()) if need else 0.0,
        "max_rel_diff": float(rel.max()) if need else 0.0,
        "atol": atol, "rtol": rtol, "eager_ms": eager_ms, "graph_ms": graph_ms,
        "graph_over_eager": graph_ms / eager_ms if eager_ms > 0 else 0.0,
        "eager_over_graph": eager_ms / graph_ms if graph_ms > 0 else 0.0,
    }
    report["winner"] = "graph" if graph_ms < eager_ms else ("eager" if eager_ms < graph_ms else "tie")
    return report


def clear_attention_session_cache():
    _core.clear_attention2d_session_cache()


def clear_conv_attention_graph_cache():
    _core._check(_core._lib().lcConvAttentionGraphCacheClear())


# legacy-prefixed names of the top-level module (bind_integrated.cpp:959-966)
lightning_conv_relu_nchw = conv_relu_nchw
lightning_attention = attention
lightning_conv_attention_torchstrong_nchw = conv_attention_torchstrong_nchw
lightning_conv_attention_torchstrong_nchw_ab_report = conv_attention_torchstrong_nchw_ab_report
_ = N
