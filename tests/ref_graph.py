"""ctypes wrapper of the reference GraphIR in oracle/_ref/libref.so (the
reference's own include/lightning_core/core/graph.hpp compiled by
oracle/Makefile's `ref` target) plus a builder that makes the same graph in
the reference and in lightning_core.

Test infrastructure only: the reference is the checker of the hip backend's
planner and executor, never part of the product.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref.so")

_P, _S, _I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
_lib = None


def available() -> bool:
    return os.path.exists(REF_SO)


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(REF_SO)
        L.ref_graph_create.restype = _P
        L.ref_graph_destroy.argtypes = [_P]
        L.ref_graph_add_tensor.argtypes = [_P, ctypes.POINTER(ctypes.c_int64), _S, _I, _I, ctypes.c_char_p, _I,
                                           ctypes.POINTER(_S)]
        L.ref_graph_add_node.argtypes = [_P, ctypes.c_char_p, ctypes.POINTER(_S), _S, ctypes.POINTER(_S), _S,
                                         ctypes.POINTER(_S), _S, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                         ctypes.POINTER(ctypes.c_int64), _S]
        L.ref_graph_call.argtypes = [_P, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_S), ctypes.POINTER(_P),
                                     ctypes.POINTER(_S), _S]
        L.ref_graph_report.argtypes = [_P, ctypes.c_char_p, _S]
        L.ref_graph_report.restype = _S
        _lib = L
    return _lib


# reference runtime::Status -> the status string both sides report
STATUS = {0: "success", 1: "not initialized", 2: "invalid value", 3: "out of memory", 4: "not supported",
          5: "driver error", 6: "unknown error"}


def _ids(xs):
    xs = [int(x) for x in xs]
    return (_S * max(len(xs), 1))(*xs), len(xs)


class RefGraph:
    def __init__(self):
        self.L = lib()
        self.h = self.L.ref_graph_create()

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_graph_destroy(self.h)
            self.h = None

    def add_tensor(self, shape, dtype="float32", layout="contiguous", name="", constant=False):
        dims = (ctypes.c_int64 * max(len(shape), 1))(*shape)
        out = _S(0)
        st = self.L.ref_graph_add_tensor(self.h, dims, len(shape), int(dtype == "float64"),
                                         int(layout == "strided"), name.encode(), int(constant), ctypes.byref(out))
        return st, out.value

    def add_node(self, op, inputs, outputs, control_deps=(), name="", attributes=None):
        attributes = dict(attributes or {})
        (ia, ni), (oa, no), (da, nd) = _ids(inputs), _ids(outputs), _ids(control_deps)
        keys = [k.encode() for k in attributes]
        ka = (ctypes.c_char_p * max(len(keys), 1))(*keys)
        va = (ctypes.c_int64 * max(len(keys), 1))(*attributes.values())
        return self.L.ref_graph_add_node(self.h, op.encode(), ia, ni, oa, no, da, nd, name.encode(), ka, va,
                                         len(keys))

    def call(self, what, options=None, feeds=None):
        """(status, report) of one reference call."""
        opts = ";".join(f"{k}={_fmt(v)}" for k, v in (options or {}).items())
        feeds = {int(k): np.ascontiguousarray(v, np.float32).reshape(-1) for k, v in (feeds or {}).items()}
        n = len(feeds)
        fid = (_S * max(n, 1))(*feeds.keys())
        fpt = (_P * max(n, 1))(*[a.ctypes.data for a in feeds.values()])
        fsz = (_S * max(n, 1))(*[a.size for a in feeds.values()])
        st = self.L.ref_graph_call(self.h, what.encode(), opts.encode(), fid, fpt, fsz, n)
        assert st >= 0, f"reference shim rejected {what} / {opts}"
        size = self.L.ref_graph_report(self.h, None, 0)
        buf = ctypes.create_string_buffer(size)
        self.L.ref_graph_report(self.h, buf, size)
        return st, json.loads(buf.value.decode())


def _fmt(v):
    if isinstance(v, bool):
        return "1" if v else "0"
    if isinstance(v, float):
        return repr(v)
    return str(v)


def registry():
    g = RefGraph()
    st, rep = g.call("registry")
    assert st == 0
    return rep
