"""GraphIR planner parity with the reference (CPU only, no GPU needed).

The reference's own GraphIR (include/lightning_core/core/graph.hpp, compiled
into oracle/_ref/libref.so) and the hip backend's restatement
(csrc/graph.cpp) get the same graphs and the same calls; their reports must
match field for field: validation issues and status, add-time errors, the
planner's steps / groups / sync boundaries and fallback reasons, the plan
summary with its cost telemetry and plan-cache counters, and the fusion
report with eligibility reasons and cost-model estimates.  Graphs come from a
seeded generator that builds the four fusion patterns, plain chains and
broken graphs (bad shapes, aliasing, constant outputs, several writers,
unknown attributes, strided layouts, float64 where the schema refuses it).

The comparison runs where no hip device is visible, so each node's candidate
devices are the reference's (cpu); hip-only behaviour (conv2d_nchw3x3s1p1,
hip placement) is covered by the tests at the end of this file.
"""
import random

import numpy as np
import pytest

import lightning_core as lc
import ref_graph

pytestmark = pytest.mark.skipif(not ref_graph.available(), reason="oracle/_ref/libref.so not built")

HIP_ONLY_SUMMARY_KEYS = ("hip_nodes", "hip_groups")


def _no_hip():
    if lc.is_hip_available():
        pytest.skip("planner parity is pinned where the candidate devices are the reference's (no hip device)")


def _summary(s):
    return {k: v for k, v in s.items() if k not in HIP_ONLY_SUMMARY_KEYS}


def _close(a, b, path="$"):
    """Structural equality; floats to 1e-12 relative (both sides compute in
    double with the same expressions)."""
    if isinstance(a, dict):
        assert isinstance(b, dict) and set(a) == set(b), f"{path}: keys {sorted(a)} != {sorted(b)}"
        for k in a:
            _close(a[k], b[k], f"{path}.{k}")
    elif isinstance(a, list):
        assert isinstance(b, list) and len(a) == len(b), f"{path}: {a} != {b}"
        for i, (x, y) in enumerate(zip(a, b)):
            _close(x, y, f"{path}[{i}]")
    elif isinstance(a, float) or isinstance(b, float):
        assert a is not None and b is not None, f"{path}: {a} != {b}"
        assert abs(a - b) <= 1e-12 * max(1.0, abs(a), abs(b)), f"{path}: {a} != {b}"
    else:
        assert a == b, f"{path}: {a!r} != {b!r}"


def _norm(x):
    """Our reports with the hip-only summary keys removed, recursively."""
    if isinstance(x, dict):
        return {k: _norm(v) for k, v in x.items() if k not in HIP_ONLY_SUMMARY_KEYS}
    if isinstance(x, list):
        return [_norm(v) for v in x]
    return x


class Both:
    """Builds one graph in the reference and in lightning_core."""

    def __init__(self):
        self.ref = ref_graph.RefGraph()
        self.ours = lc.GraphIR()

    def tensor(self, shape, dtype="float32", layout="contiguous", name="", constant=False):
        st, rid = self.ref.add_tensor(shape, dtype, layout, name, constant)
        try:
            oid = self.ours.add_tensor(shape, dtype, layout, name, constant)
            ost = 0
        except RuntimeError as e:
            ost, oid = e.status, None
        assert st == ost, f"add_tensor{shape}: reference {st}, ours {ost}"
        assert st != 0 or rid == oid
        return rid if st == 0 else None

    def node(self, op, ins, outs, deps=(), name="", attrs=None):
        st = self.ref.add_node(op, ins, outs, deps, name, attrs)
        try:
            self.ours.add_node(op, ins, outs, deps, name, attrs)
            ost = 0
        except RuntimeError as e:
            ost = e.status
        assert st == ost, f"add_node {op} {ins}->{outs} deps={deps}: reference {st}, ours {ost}"
        return st


def _ours(fn, *a, **k):
    try:
        return 0, fn(*a, **k)
    except RuntimeError as e:
        return e.status, None


def _attr_runs_sorted(report):
    """The reference keeps a node's attributes in an unordered_map, so the
    order of several attribute_unsupported issues of one node is unspecified:
    sort each such run."""
    out, run = [], []
    for issue in report["issues"] + [None]:
        if issue is not None and issue["reason_code"] == "attribute_unsupported" and \
                (not run or run[-1]["node_id"] == issue["node_id"]):
            run.append(issue)
            continue
        out += sorted(run, key=lambda i: i["message"])
        run = []
        if issue is not None:
            if issue["reason_code"] == "attribute_unsupported":
                run = [issue]
            else:
                out.append(issue)
    return dict(report, issues=out)


def compare_validation(b):
    st, ref = b.ref.call("validate")
    ours = b.ours.validate_report()
    _close(_attr_runs_sorted(ref), _attr_runs_sorted(ours))
    return st


def compare_plans(b, rng):
    """plan / plan_groups / plan_summary / fusion_report under several option
    sets, in the same order on both sides (the plan cache sees the same
    sequence), plus the cache statistics after each call."""
    for dev in ("cpu", "cuda", "metal"):
        st, ref = b.ref.call("plan", {"preferred_device": dev})
        ost, ours = _ours(b.ours.plan, dev)
        assert st == ost
        if st == 0:
            _close(ref, ours)
    for _ in range(4):
        opts = random_options(rng)
        for what in ("plan_groups", "plan_summary", "fusion_report", "plan_groups"):
            st, ref = b.ref.call(what, opts)
            dev = opts.get("preferred_device", "metal")
            kw = {k: v for k, v in opts.items() if k != "preferred_device"}
            ost, ours = _ours(getattr(b.ours, what), dev, **kw)
            assert st == ost, f"{what} {opts}: reference {st}, ours {ost}"
            if st == 0:
                _close(ref, _norm(ours))
            _, rs = b.ref.call("cache_stats")
            _close(rs, b.ours.plan_cache_stats())
    b.ref.call("clear_cache")
    b.ours.clear_plan_cache()
    _, rs = b.ref.call("cache_stats")
    _close(rs, b.ours.plan_cache_stats())


def random_options(rng):
    o = {"preferred_device": rng.choice(["cpu", "cuda", "metal"])}
    if rng.random() < 0.5:
        o["sync_mode"] = rng.choice(["auto", "always", "never"])
    for key in ("trace_sync_boundary", "group_by_backend_capability", "separate_fallback_segments",
                "insert_sync_on_device_change", "enable_fusion_v1", "enable_fusion_pass_conv",
                "enable_fusion_pass_matmul", "enable_fusion_pass_attention", "enable_fusion_pass_attention_qkv",
                "enable_fusion_cost_model_v1", "enable_fusion_cost_model_v2", "enable_plan_cache"):
        if rng.random() < 0.25:
            o[key] = rng.random() < 0.5
    if rng.random() < 0.3:
        o["fusion_pass_order"] = rng.choice(["attention_qkv,attention,matmul,conv", "matmul", " Conv , bogus ,",
                                             "attention,attention", ""])
    if rng.random() < 0.3:
        o["cost_profile_signature"] = rng.choice(["default", "metal_apple_silicon", "cuda_generic", "cpu_generic",
                                                  " CPU_Generic ", "unknown_profile", "auto"])
    if rng.random() < 0.3:
        o["fusion_cost_min_speedup"] = rng.choice([1.0, 1.01, 1.5, 3.0, 50.0])
    for key, vals in (("cost_launch_overhead_ns", [0.0, 500.0, 12000.0]),
                      ("cost_sync_boundary_ns", [100.0, 2500.0, 90000.0]),
                      ("cost_transfer_overhead_ns", [0.0, 4000.0, 1e6]),
                      ("cost_matmul_per_mac_ns", [0.0035, 1.0]),
                      ("planner_cost_weight_preference", [0.0, 1.0, 5.0]),
                      ("planner_cost_weight_boundary", [0.0, 1.0, 2.0])):
        if rng.random() < 0.15:
            o[key] = rng.choice(vals)
    return o


def random_graph(rng):
    """A graph of 1-7 nodes built from the four fusion patterns and single
    ops, then (sometimes) broken in one of the ways validation reports."""
    b = Both()
    big = rng.random() < 0.2  # shapes that make the cost model reject fusions
    dim = (lambda: rng.choice([1024, 2048, 4096])) if big else (lambda: rng.randint(1, 9))
    dt = "float64" if rng.random() < 0.1 else "float32"

    def t(shape, **kw):
        kw.setdefault("dtype", dt)
        return b.tensor(shape, **kw)

    for _ in range(rng.randint(1, 3)):
        kind = rng.choice(["mm_bias_relu", "attn_proj", "qkv_attn_proj", "conv", "binary", "relu", "mm"])
        if kind in ("mm_bias_relu", "mm"):
            m, k, n = dim(), dim(), dim()
            a, w, c = t([m, k]), t([k, n]), t([m, n])
            b.node("matmul", [a, w], [c])
            if kind == "mm_bias_relu":
                bias, s, r = t([m, n]), t([m, n]), t([m, n])
                b.node("vector_add", [c, bias] if rng.random() < 0.7 else [bias, c], [s])
                b.node("relu", [s], [r])
        elif kind == "attn_proj":
            s_, d, e = dim(), dim(), dim()
            q, k_, v, o = t([s_, d]), t([s_, d]), t([s_, d]), t([s_, d])
            b.node("attention_forward", [q, k_, v], [o], attrs={"causal": rng.randint(0, 1)} if rng.random() < 0.3
                   else None)
            w, p = t([d, e]), t([s_, e])
            b.node("matmul", [o, w], [p])
        elif kind == "qkv_attn_proj":
            s_, d, e = dim(), dim(), dim()
            x = t([1, rng.randint(1, 4), dim(), dim()])
            q, k_, v, o = t([s_, d]), t([s_, d]), t([s_, d]), t([s_, d])
            b.node("qkv_pack_repeat", [x], [q, k_, v])
            b.node("attention_forward", [q, k_, v], [o])
            w, p = t([d, e]), t([s_, e])
            b.node("matmul", [o, w], [p])
        elif kind == "conv":
            n, c, h, w_ = rng.randint(1, 2), rng.randint(1, 3), rng.randint(3, 9), rng.randint(3, 9)
            attrs = {}
            for key, vals in (("stride_h", [1, 2]), ("stride_w", [1, 2]), ("pad_h", [0, 1]), ("pad_w", [0, 1]),
                              ("apply_relu", [0, 1])):
                if rng.random() < 0.4:
                    attrs[key] = rng.choice(vals)
            sh, sw = attrs.get("stride_h", 1), attrs.get("stride_w", 1)
            ph, pw = attrs.get("pad_h", 0), attrs.get("pad_w", 0)
            oc = rng.randint(1, 4)
            x, wt = t([n, c, h, w_]), t([oc, c, 3, 3])
            ins = [x, wt] + ([t([oc])] if rng.random() < 0.5 else [])
            y = t([n, oc, (h + 2 * ph - 3) // sh + 1, (w_ + 2 * pw - 3) // sw + 1])
            b.node("conv2d_nchw3x3", ins, [y], attrs=attrs)
            if rng.random() < 0.5:
                r = t([n, oc, (h + 2 * ph - 3) // sh + 1, (w_ + 2 * pw - 3) // sw + 1])
                b.node("relu", [y], [r])
        elif kind == "binary":
            shape = [dim(), dim()]
            a, c, o = t(shape), t(shape), t(shape)
            b.node(rng.choice(["vector_add", "matrix_sub", "matrix_div"]), [a, c], [o])
        else:
            shape = [dim() for _ in range(rng.randint(1, 3))]
            a, o = t(shape), t(shape)
            b.node("relu", [a], [o])

    n_t, n_n = b.ours.num_tensors(), b.ours.num_nodes()
    if rng.random() < 0.4 and n_n:
        breakage = rng.choice(["shape", "alias", "constant", "writers", "attr", "layout", "rank", "deps", "f64",
                               "reuse"])
        if breakage == "shape":
            a, c, o = t([2, 3]), t([4, 5]), t([2, 5])
            b.node("matmul", [a, c], [o])
        elif breakage == "alias":
            a = t([3, 3])
            b.node("relu", [a], [a])
        elif breakage == "constant":
            a, o = t([3]), t([3], constant=True)
            b.node("relu", [a], [o])
        elif breakage == "writers":
            a, o = t([3]), t([3])
            b.node("relu", [a], [o])
            b.node("relu", [a], [o])
        elif breakage == "attr":
            a, o = t([3]), t([3])
            b.node("relu", [a], [o], attrs={"alpha": 1, "beta": 2} if rng.random() < 0.3 else {"alpha": 1})
        elif breakage == "layout":
            a, o = t([3, 3], layout="strided"), t([3, 3])
            b.node("relu", [a], [o])
        elif breakage == "rank":
            a, c, o = t([2, 3, 1]), t([3, 4]), t([2, 4])
            b.node("matmul", [a, c], [o])
        elif breakage == "deps":
            a, o = t([3]), t([3])
            b.node("relu", [a], [o], deps=[0])
            b.node("relu", [a], [t([3])], deps=[n_n + 5])  # refused at add time on both sides
        elif breakage == "f64":
            q = t([4, 4], dtype="float64")
            b.node("attention_forward", [q, q, q], [t([4, 4], dtype="float64")])
        else:
            # add-time errors: out-of-range ids, wrong arity, unknown op handled in Python
            b.node("relu", [n_t + 100], [0])
            b.node("matmul", [0], [0])
    return b


@pytest.mark.parametrize("seed", range(150))
def test_planner_matches_reference(seed):
    _no_hip()
    rng = random.Random(1000 + seed)
    for _ in range(5):
        b = random_graph(rng)
        st = compare_validation(b)
        compare_plans(b, rng)
        if st != 0:
            for what in ("plan_groups", "fusion_report"):
                rs, _ = b.ref.call(what, {"preferred_device": "cpu"})
                os_, _ = _ours(getattr(b.ours, what), "cpu")
                assert rs == os_ == st


def test_registry_matches_reference():
    ref = {s["op"]: s for s in ref_graph.registry()}
    ours = {s["op"]: s for s in lc.graph_registry_schemas()}
    assert set(ref) == set(ours) and lc.graph_registry_size() == len(ref) == 9
    for op, r in ref.items():
        o = dict(ours[op])
        assert o.pop("supports_hip") is True
        r = dict(r)
        assert set(r.pop("allowed_attributes")) == set(o.pop("allowed_attributes"))
        _close(r, o, op)
    assert lc.graph_validation_passes() == ["schema_contract", "topology", "alias_lifetime", "layout_flow",
                                            "backend_capability"]


def test_fusion_cost_model_reject_and_pass():
    """A 64 x 10^6 x 64 matmul + bias + relu: the fused estimate saves
    launches that are small next to the GEMM (speedup ~1.001), so the v1 cost
    model rejects it at the default 1.01 threshold and accepts it at 1.0
    (graph.hpp:2152-2182).  Planning only: nothing is allocated."""
    _no_hip()
    b = Both()
    a, w, c = b.tensor([64, 1000000]), b.tensor([1000000, 64]), b.tensor([64, 64])
    bias, s, r = b.tensor([64, 64]), b.tensor([64, 64]), b.tensor([64, 64])
    b.node("matmul", [a, w], [c])
    b.node("vector_add", [c, bias], [s])
    b.node("relu", [s], [r])
    reports = {}
    for thr in (1.01, 1.0):
        _, ref = b.ref.call("fusion_report", {"preferred_device": "cpu", "fusion_cost_min_speedup": thr})
        ours = b.ours.fusion_report("cpu", fusion_cost_min_speedup=thr)
        _close(ref, ours)
        reports[thr] = ours[0]
    assert not reports[1.01]["fused"] and reports[1.01]["reason"].startswith("cost_model_reject(speedup=1.00")
    assert reports[1.0]["fused"] and reports[1.0]["reason"].startswith("cost_model_pass(speedup=1.00")


def test_add_time_errors_match_reference():
    b = Both()
    assert b.tensor([0, 3]) is None          # a zero dimension
    assert b.tensor([]) is None              # no dimension
    x = b.tensor([2, 2])
    assert b.node("relu", [x, x], [x]) != 0  # arity
    assert b.node("relu", [7], [x]) != 0     # tensor id out of range
    assert b.node("relu", [x], [x], deps=[0]) != 0  # dependency on a later node
    with pytest.raises(ValueError, match="op must be one of"):
        b.ours.add_node("softmax", [x], [x])
    with pytest.raises(ValueError, match="dtype must be"):
        b.ours.add_tensor([1], dtype="int8")
    with pytest.raises(ValueError, match="layout must be"):
        b.ours.add_tensor([1], layout="blocked")
    with pytest.raises(ValueError, match="sync_mode must be"):
        b.ours.plan_groups("cpu", sync_mode="sometimes")
    with pytest.raises(TypeError, match="unexpected planner option"):
        b.ours.plan_groups("cpu", enable_fusion_v2=True)


# ---- hip-specific behaviour (no reference counterpart) ---------------------------

def test_s1p1_conv_is_hip_capable():
    """conv2d_nchw3x3s1p1 is Metal-only in the reference (graph.hpp:268-287):
    on a Linux build it fails validation with backend_unavailable.  The hip
    column makes it valid here; its planning then needs a hip device."""
    g = lc.GraphIR()
    x, w, y, r = g.add_tensor([1, 2, 5, 5]), g.add_tensor([3, 2, 3, 3]), g.add_tensor([1, 3, 5, 5]), \
        g.add_tensor([1, 3, 5, 5])
    g.add_node("conv2d_nchw3x3s1p1", [x, w], [y])
    g.add_node("relu", [y], [r])
    assert g.validate_report()["ok"]
    ref = ref_graph.RefGraph()
    for shape in ([1, 2, 5, 5], [3, 2, 3, 3], [1, 3, 5, 5], [1, 3, 5, 5]):
        ref.add_tensor(shape)
    ref.add_node("conv2d_nchw3x3s1p1", [0, 1], [2])
    _, rep = ref.call("validate")
    assert not rep["ok"] and rep["issues"][0]["reason_code"] == "backend_unavailable"
    if lc.is_hip_available():
        steps = g.plan("cpu")
        assert steps[0]["assigned_device"] == "hip" and steps[0]["fallback_reason_code"] == \
            "fallback_preferred_unsupported"
        fr = g.fusion_report("hip")
        assert fr[0]["pattern"] == "conv_relu_v1" and fr[0]["fused"]
    else:
        with pytest.raises(RuntimeError, match="not supported"):
            g.plan("cpu")


def test_float64_nodes_plan_off_hip_and_execution_refuses():
    g = lc.GraphIR()
    a, b_, c = g.add_tensor([2, 2], "float64"), g.add_tensor([2, 2], "float64"), g.add_tensor([2, 2], "float64")
    g.add_node("matmul", [a, b_], [c])
    steps = g.plan("hip")
    assert steps[0]["assigned_device"] == "cpu"
    assert steps[0]["fallback"] and steps[0]["fallback_reason_code"] == "fallback_preferred_unsupported"
    with pytest.raises(RuntimeError, match="not supported"):
        g.execute_f64({a: np.eye(2), b_: np.eye(2)})
    # float32 feeds for float64 tensors: invalid value, as the reference's
    # validateExecutionValues (graph.hpp:2810-2830) has it
    with pytest.raises(RuntimeError, match="invalid value"):
        g.execute_f32({a: np.eye(2), b_: np.eye(2)})


def test_cpu_placed_float32_graph_is_refused_before_any_launch():
    g = lc.GraphIR()
    a, o = g.add_tensor([4]), g.add_tensor([4])
    g.add_node("relu", [a], [o])
    with pytest.raises(RuntimeError, match="not supported: .*planned on cpu"):
        g.execute_f32({a: np.ones(4)}, preferred_device="cpu")


def test_hip_profile_and_summary_keys():
    g = lc.GraphIR()
    a, o = g.add_tensor([4]), g.add_tensor([4])
    g.add_node("relu", [a], [o])
    s = g.plan_summary("hip")["summary"]
    assert s["cost_profile_signature"] == "hip_mi355x"
    assert "hip_nodes" in s and "hip_groups" in s
    if not lc.is_hip_available():
        # hip unavailable: the preferred device falls back to the CPU
        assert s["cpu_nodes"] == 1 and s["total_fallback_nodes"] == 1
