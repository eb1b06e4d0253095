"""GraphIR on hip: the reference's graph surface (python/bindings/bind_graph.cpp)
over the C ABI's lcGraph* entry points.

Same class, method, argument and report-key names as the reference module;
the planner options keep the reference's keyword names and defaults except
``preferred_device``, which defaults to "hip" here.  Every node runs on the
GPU: ``execute_f32`` on a plan that places a node elsewhere (float64
tensors, preferred_device "cpu") raises with status "not supported"; there is
no CPU compute path.  Reports are the reference's dicts and lists; plan
summaries add ``hip_nodes`` / ``hip_groups``.
"""
from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _native as N
from ._core import _check, _lib, LightningCoreError

__all__ = ["GraphIR", "graph_validation_passes", "graph_registry_size", "graph_registry_schemas",
           "graph_registry_schema"]

_OPS = ("matmul", "vector_add", "matrix_sub", "matrix_div", "attention_forward", "conv2d_nchw3x3",
        "conv2d_nchw3x3s1p1", "qkv_pack_repeat", "relu")
_OP_ERROR = ("op must be one of: matmul, vector_add, matrix_sub, matrix_div, attention_forward, conv2d_nchw3x3, "
             "conv2d_nchw3x3s1p1, qkv_pack_repeat, relu")
_DTYPES = {"float32": 0, "float64": 1}
_LAYOUTS = {"contiguous": 0, "strided": 1}
_DEVICES = {"cpu": N.LC_DEVICE_CPU, "cuda": N.LC_DEVICE_CUDA, "metal": N.LC_DEVICE_METAL, "hip": N.LC_DEVICE_HIP}
_SYNC_MODES = {"auto": 0, "always": 1, "never": 2}

# The reference's planner keywords and defaults (bind_graph.cpp:508-533),
# preferred_device aside.
_PLANNER_DEFAULTS = {
    "sync_mode": "auto",
    "trace_sync_boundary": False,
    "group_by_backend_capability": True,
    "separate_fallback_segments": True,
    "insert_sync_on_device_change": True,
    "enable_fusion_v1": True,
    "enable_fusion_pass_conv": True,
    "enable_fusion_pass_matmul": True,
    "enable_fusion_pass_attention": True,
    "enable_fusion_pass_attention_qkv": True,
    "fusion_pass_order": "conv,matmul,attention,attention_qkv",
    "enable_fusion_cost_model_v1": True,
    "enable_fusion_cost_model_v2": True,
    "enable_plan_cache": True,
    "fusion_cost_min_speedup": 1.01,
    "cost_profile_signature": "auto",
    "cost_launch_overhead_ns": 12000.0,
    "cost_transfer_overhead_ns": 4000.0,
    "cost_sync_boundary_ns": 2500.0,
    "cost_elementwise_per_element_ns": 0.50,
    "cost_matmul_per_mac_ns": 0.0035,
    "cost_conv_per_mac_ns": 0.0022,
    "planner_cost_weight_compute": 1.0,
    "planner_cost_weight_boundary": 1.0,
    "planner_cost_weight_preference": 1.0,
}


def _device(name: str) -> int:
    try:
        return _DEVICES[name]
    except KeyError:
        raise ValueError("device must be 'cpu', 'cuda', 'metal', or 'hip'") from None


def _options(preferred_device, kwargs):
    unknown = set(kwargs) - set(_PLANNER_DEFAULTS)
    if unknown:
        raise TypeError(f"unexpected planner option(s): {', '.join(sorted(unknown))}")
    v = dict(_PLANNER_DEFAULTS, **kwargs)
    if v["sync_mode"] not in _SYNC_MODES:
        raise ValueError("sync_mode must be 'auto', 'always', or 'never'")
    o = N.GraphPlannerOptions()
    o.preferred_device = _device(preferred_device)
    o.sync_mode = _SYNC_MODES[v["sync_mode"]]
    for key in ("trace_sync_boundary", "group_by_backend_capability", "separate_fallback_segments",
                "insert_sync_on_device_change", "enable_fusion_v1", "enable_fusion_pass_conv",
                "enable_fusion_pass_matmul", "enable_fusion_pass_attention", "enable_fusion_pass_attention_qkv",
                "enable_fusion_cost_model_v1", "enable_fusion_cost_model_v2", "enable_plan_cache"):
        setattr(o, key, int(bool(v[key])))
    # the strings live as long as the options struct (kept by the caller)
    o._strings = (str(v["fusion_pass_order"]).encode(), str(v["cost_profile_signature"]).encode())
    o.fusion_pass_order, o.cost_profile_signature = o._strings
    for key in ("fusion_cost_min_speedup", "cost_launch_overhead_ns", "cost_transfer_overhead_ns",
                "cost_sync_boundary_ns", "cost_elementwise_per_element_ns", "cost_matmul_per_mac_ns",
                "cost_conv_per_mac_ns", "planner_cost_weight_compute", "planner_cost_weight_boundary",
                "planner_cost_weight_preference"):
        setattr(o, key, float(v[key]))
    return o


def _json_call(fn, *args):
    """Calls fn(*args, buf, cap, &needed) twice: size, then copy."""
    need = ctypes.c_size_t(0)
    _check(fn(*args, None, 0, ctypes.byref(need)))
    buf = ctypes.create_string_buffer(need.value)
    _check(fn(*args, buf, need.value, ctypes.byref(need)))
    return json.loads(buf.value.decode())


def graph_validation_passes():
    """bind_graph.cpp:309-317."""
    return ["schema_contract", "topology", "alias_lifetime", "layout_flow", "backend_capability"]


def graph_registry_schemas():
    """bind_graph.cpp:323-330 (each schema also carries supports_hip)."""
    return _json_call(_lib().lcGraphRegistry)


def graph_registry_size():
    return len(graph_registry_schemas())


def graph_registry_schema(op: str):
    if op not in _OPS:
        raise ValueError(_OP_ERROR)
    for s in graph_registry_schemas():
        if s["op"] == op:
            return s
    raise RuntimeError("operator schema not found")


class GraphIR:
    """lightning_core.GraphIR (bind_graph.cpp:340-906) on the hip backend."""

    def __init__(self):
        self._lib = _lib()
        h = ctypes.c_void_p()
        _check(self._lib.lcGraphCreate(ctypes.byref(h)))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.lcGraphDestroy(h)
            self._h = None

    def _report(self):
        return _json_call(self._lib.lcGraphReport, self._h)

    # --- building ---------------------------------------------------------
    def add_tensor(self, shape, dtype="float32", layout="contiguous", name="", constant=False):
        if dtype not in _DTYPES:
            raise ValueError("dtype must be 'float32' or 'float64'")
        if layout not in _LAYOUTS:
            raise ValueError("layout must be 'contiguous' or 'strided'")
        dims = (ctypes.c_int64 * max(len(shape), 1))(*[int(d) for d in shape])
        out = ctypes.c_size_t(0)
        _check(self._lib.lcGraphAddTensor(self._h, dims, len(shape), _DTYPES[dtype], _LAYOUTS[layout],
                                          str(name).encode(), int(bool(constant)), ctypes.byref(out)))
        return out.value

    def add_node(self, op, inputs, outputs, control_deps=(), name="", attributes=None):
        if op not in _OPS:
            raise ValueError(_OP_ERROR)
        attributes = dict(attributes or {})

        def ids(xs):
            xs = [int(x) for x in xs]
            return (ctypes.c_size_t * max(len(xs), 1))(*xs), len(xs)

        (ia, ni), (oa, no), (da, nd) = ids(inputs), ids(outputs), ids(control_deps)
        keys = [str(k).encode() for k in attributes]
        ka = (ctypes.c_char_p * max(len(keys), 1))(*keys)
        va = (ctypes.c_int64 * max(len(keys), 1))(*[int(v) for v in attributes.values()])
        _check(self._lib.lcGraphAddNode(self._h, op.encode(), ia, ni, oa, no, da, nd, str(name).encode(), ka, va,
                                        len(keys)))

    # --- inspection -------------------------------------------------------
    def validate(self):
        _check(self._lib.lcGraphValidate(self._h))

    def validate_report(self):
        self._lib.lcGraphValidate(self._h)  # the report is written whatever the outcome
        return self._report()

    def _counts(self):
        t, n = ctypes.c_size_t(0), ctypes.c_size_t(0)
        _check(self._lib.lcGraphCounts(self._h, ctypes.byref(t), ctypes.byref(n)))
        return t.value, n.value

    def num_tensors(self):
        return self._counts()[0]

    def num_nodes(self):
        return self._counts()[1]

    def clear_plan_cache(self):
        _check(self._lib.lcGraphClearPlanCache(self._h))

    def plan_cache_stats(self):
        h, m = ctypes.c_size_t(0), ctypes.c_size_t(0)
        _check(self._lib.lcGraphPlanCacheStats(self._h, ctypes.byref(h), ctypes.byref(m)))
        total = h.value + m.value
        return {"hits": h.value, "misses": m.value, "hit_rate_pct": 100.0 * h.value / total if total else 0.0}

    def _describe(self):
        _check(self._lib.lcGraphDescribe(self._h))
        return self._report()

    def tensors(self):
        return [{k: t[k] for k in ("name", "constant", "shape", "dtype", "layout")}
                for t in self._describe()["tensors"]]

    def nodes(self):
        return self._describe()["nodes"]

    # --- planning ---------------------------------------------------------
    def plan(self, preferred_device="hip"):
        _check(self._lib.lcGraphPlanForDevice(self._h, _device(preferred_device)))
        return self._report()

    def plan_groups(self, preferred_device="hip", **options):
        o = _options(preferred_device, options)
        _check(self._lib.lcGraphPlanGroups(self._h, ctypes.byref(o)))
        return self._report()

    def plan_summary(self, preferred_device="hip", **options):
        o = _options(preferred_device, options)
        _check(self._lib.lcGraphPlanSummary(self._h, ctypes.byref(o)))
        return self._report()

    def fusion_report(self, preferred_device="hip", **options):
        o = _options(preferred_device, options)
        _check(self._lib.lcGraphFusionReport(self._h, ctypes.byref(o)))
        return self._report()

    # --- execution --------------------------------------------------------
    def execute_f32(self, feeds, preferred_device="hip", fetch=None, **options):
        """Runs the graph on the GPU.  Returns {"values", "groups", "steps",
        "summary"}; "values" maps tensor id -> flat float32 array for every
        fed or produced tensor, as the reference does, or for the ids in
        `fetch` only (fewer downloads; a fused pattern then skips the
        intermediates nobody asked for)."""
        o = _options(preferred_device, options)
        desc = self._describe()
        feed_ids, arrays = [], []
        for tid, arr in dict(feeds).items():
            feed_ids.append(int(tid))
            arrays.append(np.ascontiguousarray(arr, dtype=np.float32).reshape(-1))
        if fetch is None:
            produced = {t for nd in desc["nodes"] for t in nd["outputs"]}
            fetch = sorted(set(feed_ids) | produced)
        fetch = [int(t) for t in fetch]
        for t in fetch:
            if t >= len(desc["tensors"]):
                raise RuntimeError("invalid value: requested tensor id out of range")
        outs = [np.empty(int(np.prod(desc["tensors"][t]["shape"])), np.float32) for t in fetch]
        nf, no = len(feed_ids), len(fetch)
        fid = (ctypes.c_size_t * max(nf, 1))(*feed_ids)
        fpt = (ctypes.c_void_p * max(nf, 1))(*[a.ctypes.data for a in arrays])
        fsz = (ctypes.c_size_t * max(nf, 1))(*[a.size for a in arrays])
        oid = (ctypes.c_size_t * max(no, 1))(*fetch)
        opt = (ctypes.c_void_p * max(no, 1))(*[a.ctypes.data for a in outs])
        _check(self._lib.lcGraphExecuteF32(self._h, ctypes.byref(o), fid, fpt, fsz, nf, oid, opt, no))
        rep = self._report()
        rep["values"] = dict(zip(fetch, outs))
        return rep

    def execute_f64(self, feeds, preferred_device="hip", **options):
        """float64 graphs are planned on the CPU, which this backend does not
        compute on."""
        _options(preferred_device, options)
        raise LightningCoreError(N.LC_NOT_SUPPORTED,
                                 "not supported: execute_f64 -- the hip backend computes graphs in float32 only")
