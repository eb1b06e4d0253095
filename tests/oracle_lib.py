"""ctypes loader for oracle/liboracle.so (the CPU checker) plus parity metrics.

Test infrastructure only.  The oracle is built by `make -C oracle` (also run
by __graft_entry__.build()).
"""
from __future__ import annotations

import ctypes
import glob
import json
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")

_P = ctypes.c_void_p
_S = ctypes.c_size_t
_I = ctypes.c_int
_F = ctypes.c_float


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


class Oracle:
    def __init__(self, lib):
        self.lib = lib
        lib.orc_attention_forward.argtypes = [_P, _P, _P, _P, _S, _S, _I]
        lib.orc_attention_forward_rows.argtypes = [_P, _P, _P, _P, _S, _S, _I, _S, _S]
        lib.orc_attention_postprocess.argtypes = [_P, _S, _F, _F, _I]
        lib.orc_attention_postprocess.restype = None
        lib.orc_attention_forward_batched.argtypes = [_P, _P, _P, _P, _S, _S, _S, _S, _I]
        lib.orc_attention_train_step.argtypes = [_P, _P, _P, _P, _P, _S, _S, _I, _F, _P]
        lib.orc_matmul.argtypes = [_P, _P, _P, _S, _S, _S]
        lib.orc_matmul_rows.argtypes = [_P, _P, _P, _S, _S, _S, _S, _S]
        lib.orc_conv2d_nchw.argtypes = [_P, _P, _P, _P] + [_S] * 11 + [_I]
        lib.orc_qkv_pack_repeat.argtypes = [_P, _S, _S, _P]
        lib.orc_qkv_pack_repeat.restype = None
        lib.orc_conv_attention_torchstrong_nchw.argtypes = [_P, _P, _P, _P] + [_S] * 13
        lib.orc_vit_block.argtypes = [_P, _P, _P, _P, _P] + [_S] * 9

    @staticmethod
    def _c(a):
        return np.ascontiguousarray(a, dtype=np.float32)

    def attention(self, q, k, v, causal=False, rows=None):
        q, k, v = self._c(q), self._c(k), self._c(v)
        s, d = q.shape
        r0, r1 = (0, s) if rows is None else rows
        out = np.zeros((r1 - r0, d), np.float32)
        st = self.lib.orc_attention_forward_rows(_ptr(q), _ptr(k), _ptr(v), _ptr(out), s, d, int(causal), r0, r1)
        assert st == 0, st
        return out

    def attention_train_step(self, q, k, v, target, lr, causal=False):
        """Returns (out, updated v, loss); the inputs are not modified."""
        q, k, target = self._c(q), self._c(k), self._c(target)
        v = self._c(v).copy()
        s, d = q.shape
        out = np.zeros((s, d), np.float32)
        loss = np.zeros(1, np.float32)
        st = self.lib.orc_attention_train_step(_ptr(q), _ptr(k), _ptr(v), _ptr(target), _ptr(out), s, d,
                                               int(causal), lr, _ptr(loss))
        assert st == 0, st
        return out, v, float(loss[0])

    def postprocess(self, out, scale, bias, relu):
        out = self._c(out).copy()
        self.lib.orc_attention_postprocess(_ptr(out), out.size, scale, bias, int(relu))
        return out

    def attention_batched(self, q, k, v, causal=False):
        q, k, v = self._c(q), self._c(k), self._c(v)
        b, h, s, d = q.shape
        out = np.zeros_like(q)
        assert self.lib.orc_attention_forward_batched(_ptr(q), _ptr(k), _ptr(v), _ptr(out), b, h, s, d,
                                                      int(causal)) == 0
        return out

    def attention_batched_rows(self, q, k, v, causal, rows):
        """Rows [r0, r1) of every (b, h) problem: result [B, H, r1-r0, D]."""
        b, h, s, d = q.shape
        r0, r1 = rows
        out = np.zeros((b, h, r1 - r0, d), np.float32)
        for bi in range(b):
            for hi in range(h):
                out[bi, hi] = self.attention(q[bi, hi], k[bi, hi], v[bi, hi], causal, rows)
        return out

    def matmul(self, a, b, rows=None):
        a, b = self._c(a), self._c(b)
        m, k = a.shape
        n = b.shape[1]
        r0, r1 = (0, m) if rows is None else rows
        out = np.zeros((r1 - r0, n), np.float32)
        assert self.lib.orc_matmul_rows(_ptr(a), _ptr(b), _ptr(out), m, k, n, r0, r1) == 0
        return out

    def conv2d(self, x, w, bias, stride=(1, 1), pad=(0, 0), relu=False):
        x, w = self._c(x), self._c(w)
        bias = None if bias is None else self._c(bias)
        bn, c, h, wd = x.shape
        oc, _, kh, kw = w.shape
        oh = (h + 2 * pad[0] - kh) // stride[0] + 1
        ow = (wd + 2 * pad[1] - kw) // stride[1] + 1
        out = np.zeros((bn, oc, oh, ow), np.float32)
        st = self.lib.orc_conv2d_nchw(_ptr(x), _ptr(w), _ptr(bias), _ptr(out), bn, c, h, wd, oc, kh, kw,
                                      stride[0], stride[1], pad[0], pad[1], int(relu))
        assert st == 0, st
        return out

    def qkv_pack_repeat(self, conv, need):
        conv = self._c(conv).ravel()
        packed = np.zeros(3 * need, np.float32)
        self.lib.orc_qkv_pack_repeat(_ptr(conv), conv.size, need, _ptr(packed))
        return packed

    def conv_attention(self, x, w, bias, seq_len, head_dim, stride=(1, 1), pad=(0, 0)):
        x, w = self._c(x), self._c(w)
        bias = None if bias is None else self._c(bias)
        bn, c, h, wd = x.shape
        oc, _, kh, kw = w.shape
        out = np.zeros((seq_len, head_dim), np.float32)
        st = self.lib.orc_conv_attention_torchstrong_nchw(_ptr(x), _ptr(w), _ptr(bias), _ptr(out), bn, c, h, wd, oc,
                                                          kh, kw, seq_len, head_dim, stride[0], stride[1], pad[0],
                                                          pad[1])
        assert st == 0, st
        return out

    def vit_block(self, x, w_conv, w_qkv, w_o, heads, rows=None):
        x, w_conv, w_qkv, w_o = self._c(x), self._c(w_conv), self._c(w_qkv), self._c(w_o)
        bn, c, h, wd = x.shape
        embed, _, patch, _ = w_conv.shape
        t = (h // patch) * (wd // patch)
        r0, r1 = (0, bn * t) if rows is None else rows
        out = np.zeros((r1 - r0, embed), np.float32)
        st = self.lib.orc_vit_block(_ptr(x), _ptr(w_conv), _ptr(w_qkv), _ptr(w_o), _ptr(out), bn, c, h, wd, patch,
                                    embed, heads, r0, r1)
        assert st == 0, st
        return out


def build():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def load() -> Oracle:
    if not os.path.exists(ORACLE_SO):
        build()
    return Oracle(ctypes.CDLL(ORACLE_SO))


def golden_cases(prefix=""):
    out = []
    for path in sorted(glob.glob(os.path.join(GOLDEN_DIR, prefix + "*.json"))):
        with open(path) as f:
            out.append(json.load(f))
    return out


def golden_input(case, key):
    v = case["inputs"][key]
    return None if v is None else np.asarray(v, dtype=np.float32)


# --- parity metrics ----------------------------------------------------------

def normwise_rel(ref, got) -> float:
    """max|got - ref| / max|ref| (the headline parity metric)."""
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    denom = max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(got - ref))) / denom


def elementwise_ok(ref, got, atol, rtol) -> bool:
    """|got - ref| <= atol + rtol*|ref| (tests/test_backend_parity.cpp:52)."""
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    return bool(np.all(np.abs(got - ref) <= atol + rtol * np.abs(ref)))
