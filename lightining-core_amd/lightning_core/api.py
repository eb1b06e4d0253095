"""lightning_core.api -- the integrated conv -> attention entry points.

Mirrors the reference's `api` submodule (python/bindings/bind_integrated.cpp:
951-1190): conv_relu_nchw[_into], attention[_into],
conv_attention_torchstrong_nchw[_into].  `execution_mode` accepts "eager" and
"graph"; both run the same on-device chain here (the reference's graph mode
falls back to eager on any planning error, bind_integrated.cpp:929-942).
"""
from __future__ import annotations

import numpy as np

from . import _core
from . import _native as N

__all__ = ["conv_relu_nchw", "conv_relu_nchw_into", "attention", "attention_into",
           "conv_attention_torchstrong_nchw", "conv_attention_torchstrong_nchw_into",
           "clear_attention_session_cache"]


def _mode(execution_mode: str):
    if execution_mode not in ("eager", "graph"):
        raise ValueError("unsupported execution mode")


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
    _core._check(_core._lib().lcConvAttentionTorchstrongNchw(
        _core._fp(x), _core._fp(w), _core._fp(b), _core._fp(out), bn, c, h, wd, oc, kh, kw, seq_len, head_dim,
        stride_h, stride_w, pad_h, pad_w, _core._parse_device(device)))


def conv_attention_torchstrong_nchw(x, w, bias, seq_len, head_dim, stride_h=1, stride_w=1, pad_h=0, pad_w=0,
                                    device="hip", execution_mode="eager"):
    """bind_integrated.cpp:1059-1098: returns a flat [seq_len*head_dim] array."""
    out = np.empty(seq_len * head_dim, np.float32)
    conv_attention_torchstrong_nchw_into(x, w, bias, out, seq_len, head_dim, stride_h, stride_w, pad_h, pad_w,
                                         device, execution_mode)
    return out


def clear_attention_session_cache():
    _core.clear_attention2d_session_cache()


# legacy-prefixed names of the top-level module (bind_integrated.cpp:959-966)
lightning_conv_relu_nchw = conv_relu_nchw
lightning_attention = attention
lightning_conv_attention_torchstrong_nchw = conv_attention_torchstrong_nchw
_ = N
