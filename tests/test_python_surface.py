"""The Python mirror's names, argument checks and runtime helpers (CPU only).

The reference's pybind module (python/bindings/bind_runtime.cpp:390-529,
bind_ops.cpp:635-888) is the model: same names, argument names, defaults and
error types.  Nothing here launches a kernel: validation runs before any
device work, and the runtime helpers only query the library.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

import lightning_core as lc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_reference_runtime_names_exist():
    for name in ("cuda_available", "metal_available", "backend_name", "memory_model_name", "runtime_sync_policy_set",
                 "runtime_sync_policy_get", "runtime_sync_apply", "runtime_sync_apply_default",
                 "runtime_backend_capabilities", "runtime_active_backend_capabilities", "runtime_backend_interfaces",
                 "runtime_active_backend_interfaces", "runtime_trace_enable", "runtime_trace_enabled",
                 "runtime_trace_clear", "runtime_trace_capacity", "runtime_trace_events", "runtime_trace_timeline",
                 "matmul", "matmul_np", "matmul_np_into", "matmul_with_policy", "matmul_np_with_policy",
                 "matmul_np_into_with_policy", "conv2d_nchw", "conv2d_nchw_into", "matmul2d", "matmul2d_into",
                 "matmul2d_resident_session", "attention2d", "attention2d_into", "attention_forward",
                 "attention_forward_with_policy", "attention2d_session", "clear_attention2d_session_cache"):
        assert callable(getattr(lc, name)), name
        assert name in lc.__all__, name


def test_availability_and_memory_model():
    assert lc.cuda_available() is False and lc.metal_available() is False
    assert lc.memory_model_name() == "native-device"


def test_sync_policy_names_roundtrip():
    old = lc.runtime_sync_policy_get()
    try:
        lc.runtime_sync_policy_set("never", trace_sync_boundary=True)
        assert lc.runtime_sync_policy_get() == {"mode": "never", "trace_sync_boundary": True}
        lc.runtime_sync_apply("never")  # no device work
        lc.runtime_sync_policy_set()
        assert lc.runtime_sync_policy_get() == {"mode": "auto", "trace_sync_boundary": False}
        with pytest.raises(ValueError, match="sync mode"):
            lc.runtime_sync_policy_set("sometimes")
        with pytest.raises(ValueError, match="sync mode"):
            lc.runtime_sync_apply("later")
    finally:
        lc.runtime_sync_policy_set(old["mode"], old["trace_sync_boundary"])


def test_interface_dicts_carry_reference_keys():
    d = lc.runtime_backend_interfaces("hip")
    assert set(d) == {"device", "capabilities", "compute", "memory", "sync", "profiler"}
    assert set(d["compute"]) == {"available", "op_dispatch_trace_surface", "driver_tag"}
    assert set(d["memory"]) == {"available", "allocator_surface", "memcpy_surface", "memory_model", "driver_tag"}
    assert set(d["sync"]) == {"available", "sync_policy_surface", "trace_sync_boundary_surface", "driver_tag"}
    assert set(d["profiler"]) == {"available", "runtime_trace_surface", "op_dispatch_trace_surface",
                                  "trace_capacity", "driver_tag"}
    active = lc.runtime_active_backend_interfaces()
    assert active["device"] == ("hip" if lc.is_hip_available() else "cpu")
    assert lc.runtime_active_backend_capabilities()["device"] == active["device"]


def test_trace_events_and_timeline():
    lc.runtime_trace_clear()
    lc.runtime_trace_enable(True)
    try:
        assert lc.runtime_trace_enabled()
        lc.backend_name()
        lc.cuda_available()
        lc.metal_available()
        lc.cuda_available()
    finally:
        lc.runtime_trace_enable(False)
    assert not lc.runtime_trace_enabled()
    assert lc.runtime_trace_capacity() == 4096
    ev = lc.runtime_trace_events()
    assert [e["type"] for e in ev] == ["backend_name", "is_cuda_available", "is_metal_available",
                                       "is_cuda_available"]
    assert all(e["status"] == "success" and e["op"] == "" and e["requested_device"] == "" for e in ev)
    t = lc.runtime_trace_timeline(group_by="type", group_sort_by="count", hotspot_top_k=2)
    assert t["event_count"] == 4 and len(t["events"]) == 4 and len(t["hotspots"]) == 2
    ts = [e["timestamp_ns"] for e in t["events"]]
    assert ts == sorted(ts) and t["events"][0]["offset_ns"] == 0
    assert t["window_ns"] == ts[-1] - ts[0]
    # gaps: delta_next of event i is delta_prev of event i + 1; the last is 0
    evs = t["events"]
    assert all(evs[i]["delta_next_ns"] == evs[i + 1]["delta_prev_ns"] for i in range(3))
    assert evs[-1]["delta_next_ns"] == 0
    assert t["groups"][0]["key"] == "is_cuda_available" and t["groups"][0]["count"] == 2
    assert sum(g["count"] for g in t["groups"]) == 4
    assert abs(sum(g["window_share_pct"] for g in t["groups"]) - 100.0) < 1e-9 or t["window_ns"] == 0
    hot = t["hotspots"]
    assert hot[0]["delta_next_ns"] >= hot[1]["delta_next_ns"]
    desc = lc.runtime_trace_timeline(event_sort_by="index", event_descending=True, group_by="op")
    assert [e["index"] for e in desc["events"]] == [3, 2, 1, 0]
    assert [g["key"] for g in desc["groups"]] == ["non_op"]
    with pytest.raises(ValueError, match="group_by"):
        lc.runtime_trace_timeline(group_by="device")
    with pytest.raises(ValueError, match="event_sort_by"):
        lc.runtime_trace_timeline(event_sort_by="name")
    lc.runtime_trace_clear()
    empty = lc.runtime_trace_timeline()
    assert empty["event_count"] == 0 and empty["window_ns"] == 0 and empty["groups"] == []


def test_matmul_policy_entries_check_sizes():
    a, b = np.ones(6, np.float32), np.ones(6, np.float32)
    with pytest.raises(ValueError, match="shape mismatch"):
        lc.matmul_with_policy(a, np.ones(5, np.float32), 2, 3, 2)
    with pytest.raises(ValueError, match="shape mismatch"):
        lc.matmul_with_policy(np.ones(7, np.float32), b, 2, 3, 2)
    with pytest.raises(ValueError, match="out"):
        lc.matmul_with_policy(a, b, 2, 3, 2, out=np.zeros(3, np.float32))
    with pytest.raises(ValueError, match="out"):
        lc.matmul_with_policy(a, b, 2, 3, 2, out=np.zeros(4, np.float64))
    with pytest.raises(ValueError, match="out"):
        lc.matmul_with_policy(a, b, 2, 3, 2, out=np.zeros((4, 2), np.float32)[:, 0])
    with pytest.raises(ValueError, match="shape mismatch"):
        lc.matmul_np_with_policy(a, np.ones(4, np.float32), 2, 3, 2)
    with pytest.raises(ValueError, match="out shape mismatch"):
        lc.matmul_np_into_with_policy(a, b, np.zeros(5, np.float32), 2, 3, 2)


def test_conv2d_nchw_into_checks():
    x = np.ones((1, 2, 5, 5), np.float32)
    w = np.ones((3, 2, 3, 3), np.float32)
    with pytest.raises(ValueError, match="out shape mismatch"):
        lc.conv2d_nchw_into(x, w, None, np.zeros((1, 3, 5, 5), np.float32))
    with pytest.raises(ValueError, match="4D"):
        lc.conv2d_nchw_into(x, w, None, np.zeros((3, 3, 3), np.float32))
    with pytest.raises(ValueError, match="bias"):
        lc.conv2d_nchw_into(x, w, np.ones(2), np.zeros((1, 3, 3, 3), np.float32))
    with pytest.raises(ValueError, match="channels"):
        lc.conv2d_nchw_into(x, np.ones((3, 1, 3, 3)), None, np.zeros((1, 3, 3, 3), np.float32))


def test_session_cache_clear_is_safe_without_sessions():
    lc.clear_attention2d_session_cache()
    lc.clear_attention2d_session_cache()


def test_build_rejects_reserved_register_clobbers(tmp_path):
    """The build turns hipcc's warning for inline asm that clobbers a reserved
    register (M0 here) into an error; the kernels pass M0 as an operand."""
    src = tmp_path / "clobber.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void k(int* p) {\n"
        "  asm volatile(\"s_mov_b32 m0, 0\" ::: \"m0\");\n"
        "  p[threadIdx.x] = 1;\n"
        "}\n")
    code = ("import sys; sys.path.insert(0, %r); import build; build.BUILD = %r; build._compile(%r)"
            % (os.path.join(ROOT, "lightining-core_amd"), str(tmp_path), str(src)))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "reserved register" in (r.stdout + r.stderr)
    kc = open(os.path.join(ROOT, "lightining-core_amd", "csrc", "kernels", "kcommon.hpp")).read()
    assert '"{m0}"' in kc and '"m0")' not in kc
