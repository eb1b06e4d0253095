"""Writes the golden fixtures in this folder from the reference's own CPU path.

The reference's CPU sources are compiled where they lie by `make -C oracle ref`
into oracle/_ref/libref.so (see oracle/Makefile and oracle/ref_shim.cpp); this
script calls that library on small inputs and stores inputs and outputs as
JSON.  It runs only in a container that has the reference tree; the fixtures
it writes are committed and are what the tests read.

Inputs: the reference's makeValue generator (tests/test_backend_parity.cpp:
12-23) for the reference's own parity cases, its known-answer inputs
(tests/test_attention.cpp:49-68, tests/test_matmul.cpp:14-50), and seeded
SplitMix64 values for odd shapes.

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "lightining-core_amd"))

from lightning_core import synth  # noqa: E402

_P = ctypes.c_void_p
_S = ctypes.c_size_t


def _load_ref():
    path = os.path.join(ROOT, "oracle", "_ref", "libref.so")
    if not os.path.exists(path):
        raise SystemExit("oracle/_ref/libref.so missing: run `make -C oracle ref` first")
    lib = ctypes.CDLL(path)
    lib.ref_attention_forward.argtypes = [_P, _P, _P, _P, _S, _S, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                          ctypes.c_int]
    lib.ref_attention_train_step.argtypes = [_P, _P, _P, _P, _P, _S, _S, ctypes.c_int, ctypes.c_float, _P]
    lib.ref_matmul.argtypes = [_P, _P, _P, _S, _S, _S]
    lib.ref_conv2d_nchw.argtypes = [_P, _P, _P, _P] + [_S] * 11 + [ctypes.c_int]
    lib.ref_conv_attention.argtypes = [_P, _P, _P, _P] + [_S] * 13
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _dump(name, params, inputs, expected):
    doc = {
        "name": name,
        "source": "reference CPU path compiled from /root/reference sources (oracle/_ref/libref.so)",
        "params": params,
        "inputs": {k: (None if v is None else [float(x) for x in np.asarray(v).ravel()]) for k, v in inputs.items()},
        "expected": [float(x) for x in np.asarray(expected).ravel()],
    }
    with open(os.path.join(HERE, name + ".json"), "w") as f:
        json.dump(doc, f, separators=(",", ":"))


def attention_case(lib, name, q, k, v, s, d, causal, scale=1.0, bias=0.0, relu=False):
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros(s * d, np.float32)
    st = lib.ref_attention_forward(_ptr(q), _ptr(k), _ptr(v), _ptr(out), s, d, int(causal), scale, bias, int(relu))
    assert st == 0, st
    _dump(name, {"op": "attention", "seq_len": s, "head_dim": d, "causal": bool(causal), "output_scale": scale,
                 "output_bias": bias, "output_relu": bool(relu)}, {"q": q, "k": k, "v": v}, out)


def train_case(lib, name, q, k, v, target, s, d, causal, lr):
    """attentionTrainStep: expected = out (s*d) ++ updated v (s*d) ++ [loss]."""
    q, k, v0, target = _f32(q), _f32(k), _f32(v), _f32(target)
    v = v0.copy()
    out = np.zeros(s * d, np.float32)
    loss = np.zeros(1, np.float32)
    st = lib.ref_attention_train_step(_ptr(q), _ptr(k), _ptr(v), _ptr(target), _ptr(out), s, d, int(causal),
                                      lr, _ptr(loss))
    assert st == 0, st
    _dump(name, {"op": "attention_train_step", "seq_len": s, "head_dim": d, "causal": bool(causal),
                 "learning_rate": lr, "expected_layout": ["out", "v", "loss"]},
          {"q": q, "k": k, "v": v0, "target": target}, np.concatenate([out.ravel(), v.ravel(), loss]))


def matmul_case(lib, name, a, b, m, k, n):
    a, b = _f32(a), _f32(b)
    out = np.zeros(m * n, np.float32)
    assert lib.ref_matmul(_ptr(a), _ptr(b), _ptr(out), m, k, n) == 0
    _dump(name, {"op": "matmul", "m": m, "k": k, "n": n}, {"a": a, "b": b}, out)


def conv_case(lib, name, x, w, bias, dims, relu):
    batch, in_c, in_h, in_w, out_c, kh, kw, sh, sw, ph, pw = dims
    x, w = _f32(x), _f32(w)
    bias = None if bias is None else _f32(bias)
    out_h = (in_h + 2 * ph - kh) // sh + 1
    out_w = (in_w + 2 * pw - kw) // sw + 1
    out = np.zeros(batch * out_c * out_h * out_w, np.float32)
    assert lib.ref_conv2d_nchw(_ptr(x), _ptr(w), _ptr(bias), _ptr(out), *dims, int(relu)) == 0
    keys = ["batch", "in_c", "in_h", "in_w", "out_c", "kh", "kw", "stride_h", "stride_w", "pad_h", "pad_w"]
    params = {"op": "conv2d_nchw", "relu": bool(relu), **dict(zip(keys, dims))}
    _dump(name, params, {"x": x, "w": w, "bias": bias}, out)


def conv_attention_case(lib, name, x, w, bias, dims, seq_len, head_dim):
    batch, in_c, in_h, in_w, out_c, kh, kw, sh, sw, ph, pw = dims
    x, w = _f32(x), _f32(w)
    bias = None if bias is None else _f32(bias)
    out = np.zeros(seq_len * head_dim, np.float32)
    assert lib.ref_conv_attention(_ptr(x), _ptr(w), _ptr(bias), _ptr(out), batch, in_c, in_h, in_w, out_c, kh, kw,
                                  seq_len, head_dim, sh, sw, ph, pw) == 0
    keys = ["batch", "in_c", "in_h", "in_w", "out_c", "kh", "kw", "stride_h", "stride_w", "pad_h", "pad_w"]
    params = {"op": "conv_attention", "seq_len": seq_len, "head_dim": head_dim, **dict(zip(keys, dims))}
    _dump(name, params, {"x": x, "w": w, "bias": bias}, out)


def main():
    lib = _load_ref()
    mv = synth.make_vec

    # tests/test_attention.cpp:49-68 known answer, and :70-92 postprocess.
    eye = np.array([1, 0, 0, 1], np.float32)
    vkat = np.array([10, 0, 0, 20], np.float32)
    attention_case(lib, "attention_kat_2x2", eye, eye, vkat, 2, 2, False)
    attention_case(lib, "attention_kat_2x2_post", eye, eye, vkat, 2, 2, False, 0.5, -2.0, True)
    # tests/test_backend_parity.cpp:158-185 inputs (S=16, D=32), plus causal.
    n = 16 * 32
    qv, kv, vv = mv(n, 0.01), mv(n, 0.009, 0.02), mv(n, 0.008, -0.01)
    attention_case(lib, "attention_makevalue_s16_d32", qv, kv, vv, 16, 32, False)
    attention_case(lib, "attention_makevalue_s16_d32_causal", qv, kv, vv, 16, 32, True)
    # Odd shapes (not multiples of any tile), seeded normal inputs.
    for s, d, causal in [(33, 20, False), (33, 20, True), (70, 64, True), (64, 128, False), (5, 3, True)]:
        q = synth.normal((s, d), seed=7, stream=1)
        k = synth.normal((s, d), seed=7, stream=2)
        v = synth.normal((s, d), seed=7, stream=3)
        attention_case(lib, f"attention_normal_s{s}_d{d}{'_causal' if causal else ''}", q, k, v, s, d, causal)

    # Train step (attentionTrainStep, src/attention.cpp:203-214): the
    # reference's makeValue inputs with a makeValue target, plus seeded odd
    # shapes, causal and not.
    n = 16 * 32
    train_case(lib, "train_attention_makevalue_s16_d32", qv, kv, vv, mv(n, 0.007, 0.03), 16, 32, False, 0.05)
    for s, d, causal, lr in [(33, 20, True, 0.1), (70, 64, False, 0.01), (64, 128, True, 0.5)]:
        q = synth.normal((s, d), seed=9, stream=1)
        k = synth.normal((s, d), seed=9, stream=2)
        v = synth.normal((s, d), seed=9, stream=3)
        t = synth.normal((s, d), seed=9, stream=4)
        train_case(lib, f"train_attention_normal_s{s}_d{d}{'_causal' if causal else ''}", q, k, v, t, s, d, causal,
                   lr)

    # tests/test_matmul.cpp:14-50 known answer; test_backend_parity.cpp:66-89.
    matmul_case(lib, "matmul_kat_2x3x2", np.arange(1, 7, dtype=np.float32), np.arange(7, 13, dtype=np.float32),
                2, 3, 2)
    matmul_case(lib, "matmul_makevalue_4x7x5", mv(28, 0.02), mv(35, 0.015, 0.01), 4, 7, 5)
    for m, k, nn in [(17, 19, 23), (65, 33, 130), (1, 77, 9)]:
        a = synth.uniform((m, k), seed=11, stream=1)
        b = synth.uniform((k, nn), seed=11, stream=2)
        matmul_case(lib, f"matmul_uniform_{m}x{k}x{nn}", a, b, m, k, nn)

    # tests/test_backend_parity.cpp:187-250 conv case (with and without ReLU).
    dims = (1, 3, 8, 8, 8, 3, 3, 1, 1, 1, 1)
    x, w, b = mv(192, 0.01, 0.05), mv(216, 0.01, -0.03), mv(8, 0.01, 0.02)
    conv_case(lib, "conv_makevalue_3x3_s1p1", x, w, b, dims, False)
    conv_case(lib, "conv_makevalue_3x3_s1p1_relu", x, w, b, dims, True)
    # Patch-embed geometry (kernel = stride = 16, no padding), small image.
    dims = (2, 3, 32, 48, 16, 16, 16, 16, 16, 0, 0)
    x = synth.uniform((2, 3, 32, 48), seed=5, lo=0.0, hi=1.0, stream=1)
    w = synth.normal((16, 3, 16, 16), seed=5, std=0.02, stream=2)
    conv_case(lib, "conv_patch16_s16_relu", x, w, None, dims, True)
    # Strided, padded, odd sizes.
    dims = (2, 2, 9, 7, 5, 3, 2, 2, 1, 1, 0)
    x = synth.normal((2, 2, 9, 7), seed=6, stream=1)
    w = synth.normal((5, 2, 3, 2), seed=6, stream=2)
    b = synth.normal((5,), seed=6, stream=3)
    conv_case(lib, "conv_normal_3x2_s2x1_p1x0_relu", x, w, b, dims, True)

    # Conv -> QKV arrange -> attention (bind_integrated.cpp:614-730): a case
    # where the conv output covers 3*S*D (flat slices) and one where it is
    # repeated (QkvPackRepeat).
    dims = (1, 3, 8, 8, 8, 3, 3, 1, 1, 1, 1)
    x, w, b = mv(192, 0.01, 0.05), mv(216, 0.01, -0.03), mv(8, 0.01, 0.02)
    conv_attention_case(lib, "conv_attention_slices_s8_d16", x, w, b, dims, 8, 16)
    conv_attention_case(lib, "conv_attention_repeat_s16_d16", x, w, b, dims, 16, 16)
    conv_attention_case(lib, "conv_attention_repeat_nobias_s24_d20", x, w, None, dims, 24, 20)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
