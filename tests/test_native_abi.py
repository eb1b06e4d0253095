"""The C-ABI library loads and keeps the reference's contracts (CPU only).

No compute runs here: these tests cover symbol exports, the frozen struct
layouts (tests/test_c_api_abi_freeze.cpp:7-36 in the reference), the dispatch
trace encoding (src/runtime.cpp:703-748), capability contracts, and the
validation that happens before any device work (null pointers, zero sizes,
unsupported devices).
"""
import ctypes
import os
import re

import numpy as np
import pytest

import lightning_core as lc
from lightning_core import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lightning_core_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lc[A-Z]\w*)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = N.load()
    names = _declared_functions()
    assert len(names) >= 70
    for name in names:
        assert hasattr(lib, name), name
    # and the ctypes binding covers exactly the declared surface
    assert set(names) == set(N.SIGNATURES)


def test_reference_c_abi_surface_present():
    # the 25 functions of the reference's lightning_core.h:113-137
    ref = ["lcMalloc", "lcFree", "lcMemcpy", "lcDeviceSynchronize", "lcGetDeviceCount",
           "lcGetPreferredDeviceForInference", "lcGetPreferredDeviceForTraining", "lcIsCudaAvailable",
           "lcIsMetalAvailable", "lcGetMemoryModel", "lcGetMemoryModelName", "lcSetDefaultSyncPolicy",
           "lcGetDefaultSyncPolicy", "lcApplySyncPolicy", "lcApplyDefaultSyncPolicy", "lcGetBackendCapabilities",
           "lcGetActiveBackendCapabilities", "lcGetBackendInterfaceContract", "lcGetActiveBackendInterfaceContract",
           "lcGetApiVersion", "lcGetApiVersionString", "lcGetStructSize", "lcCheckStructSize", "lcBackendName",
           "lcGetErrorString"]
    assert set(ref) <= set(_declared_functions())


def test_api_version_and_struct_sizes():
    lib = N.load()
    assert lc.api_version() == (0, 6, 0)
    assert lib.lcGetApiVersionString() == b"0.6.0-rc0"
    sizes = {N.LC_STRUCT_BACKEND_CAPABILITIES: N.BackendCapabilities,
             N.LC_STRUCT_COMPUTE_INTERFACE_CONTRACT: N.ComputeInterfaceContract,
             N.LC_STRUCT_MEMORY_INTERFACE_CONTRACT: N.MemoryInterfaceContract,
             N.LC_STRUCT_SYNC_INTERFACE_CONTRACT: N.SyncInterfaceContract,
             N.LC_STRUCT_PROFILER_INTERFACE_CONTRACT: N.ProfilerInterfaceContract,
             N.LC_STRUCT_BACKEND_INTERFACE_CONTRACT: N.BackendInterfaceContract}
    for sid, st in sizes.items():
        assert lib.lcGetStructSize(sid) == ctypes.sizeof(st)
        assert lib.lcCheckStructSize(sid, ctypes.sizeof(st)) == 1
        assert lib.lcCheckStructSize(sid, ctypes.sizeof(st) + 4) == 0
    assert lib.lcGetStructSize(99) == 0
    # the same sizes against the reference header itself, compiled with g++:
    # tests/test_reference_binding.py::test_reference_struct_sizes_match_the_library


def test_device_enum_appends_hip():
    assert (N.LC_DEVICE_CPU, N.LC_DEVICE_CUDA, N.LC_DEVICE_METAL, N.LC_DEVICE_HIP) == (0, 1, 2, 3)


@pytest.mark.parametrize("req", ["cpu", "cuda", "metal", "hip"])
@pytest.mark.parametrize("sel", ["cpu", "hip"])
@pytest.mark.parametrize("fb", [False, True])
def test_dispatch_detail_roundtrip(req, sel, fb):
    lib = N.load()
    dev = {"cpu": 0, "cuda": 1, "metal": 2, "hip": 3}
    enc = lib.lcEncodeRuntimeTraceDispatchDetail(dev[req], dev[sel], int(fb))
    assert enc == dev[req] | (dev[sel] << 4) | (256 if fb else 0)
    assert lc.decode_dispatch_detail(enc) == {"requested": req, "selected": sel, "fallback": fb}


def test_dispatch_detail_rejects_unknown_devices():
    assert lc.decode_dispatch_detail(0x0F) is None
    assert lc.decode_dispatch_detail(0x70) is None


def test_capability_matrix_has_hip_row():
    hip = lc.runtime_backend_capabilities("hip")
    assert hip["built"] and hip["compute_surface"] and hip["memory_model"] == "native-device"
    assert hip["available"] == lc.is_hip_available()
    for dev in ("cuda", "metal"):
        caps = lc.runtime_backend_capabilities(dev)
        assert not caps["built"] and not caps["available"]
    contract = lc.runtime_backend_interface_contract("hip")
    assert contract["compute"]["driver_tag"] == "hip.compute.dispatch"
    assert contract["profiler"]["trace_capacity"] == 4096
    assert lc.runtime_trace_event_capacity() == 4096


def test_sync_policy_roundtrip():
    lib = N.load()
    old = lib.lcGetDefaultSyncPolicy()
    try:
        assert lib.lcSetDefaultSyncPolicy(N.SyncPolicy(2, 1)) == 0
        p = lib.lcGetDefaultSyncPolicy()
        assert (p.mode, p.trace_sync_boundary) == (2, 1)
        assert lib.lcApplySyncPolicy(N.SyncPolicy(2, 0)) == 0  # never: no device work
    finally:
        lib.lcSetDefaultSyncPolicy(old)


def test_error_strings_match_reference():
    lib = N.load()
    names = ["success", "not initialized", "invalid value", "out of memory", "not supported", "driver error",
             "unknown error"]
    for code, name in enumerate(names):
        assert lib.lcGetErrorString(code).decode() == name


def test_validation_before_device_work():
    lib = N.load()
    a = np.ones(6, np.float32)
    out = np.zeros(4, np.float32)
    fp = a.ctypes.data_as(N.FP)
    # null pointers / zero dims -> invalid value (reference ops.hpp:367-370)
    assert lib.lcMatMul(None, fp, out.ctypes.data_as(N.FP), 2, 3, 2, N.LC_DEVICE_HIP) == N.LC_INVALID_VALUE
    assert lib.lcMatMul(fp, fp, out.ctypes.data_as(N.FP), 0, 3, 2, N.LC_DEVICE_HIP) == N.LC_INVALID_VALUE
    cfg = N.AttentionConfig(0, 2, 0)
    assert lib.lcAttentionForward(fp, fp, fp, fp, ctypes.byref(cfg), N.LC_DEVICE_HIP) == N.LC_INVALID_VALUE
    assert lib.lcAttentionSessionTrainRunCached(None, 0.5, 1) == N.LC_INVALID_VALUE
    # non-hip devices are served elsewhere: not supported, never a CPU fallback
    assert lib.lcMatMul(fp, fp, out.ctypes.data_as(N.FP), 2, 3, 2, N.LC_DEVICE_CPU) == N.LC_NOT_SUPPORTED
    assert lib.lcMatMul(fp, fp, out.ctypes.data_as(N.FP), 2, 3, 2, 7) == N.LC_INVALID_VALUE
    with pytest.raises(RuntimeError, match="not supported"):
        lc.matmul2d(np.ones((2, 3)), np.ones((3, 2)), device="metal")
    with pytest.raises(ValueError):
        lc.matmul2d(np.ones((2, 3)), np.ones((4, 2)))
    with pytest.raises(ValueError):
        lc.attention2d(np.ones((2, 3)), np.ones((2, 4)), np.ones((2, 3)))
    with pytest.raises(ValueError):
        lc.matmul2d(np.ones((2, 3)), np.ones((3, 2)), device="tpu")


@pytest.mark.skipif(lc.is_hip_available(), reason="checks the no-GPU behaviour")
def test_no_gpu_means_not_supported_not_fallback():
    assert lc.backend_name() == "cpu"
    with pytest.raises(RuntimeError, match="not supported"):
        lc.attention2d(np.eye(2), np.eye(2), np.eye(2), device="hip")
    with pytest.raises(RuntimeError, match="not supported"):
        lc.MatMulResidentSession(4, 4, 4, "bf16")


def test_tune_cache_header_roundtrip(tmp_path):
    p = tmp_path / "tune.csv"
    lc.matmul_reset_tuning()
    lc.tune_cache_save(str(p))
    lines = p.read_text().splitlines()
    assert lines[0] == "#lc_tune_cache,matmul,2"
    assert lines[1].startswith("#columns,m,k,n,dtype,arch,kernel")
    p.write_text("#lc_tune_cache,matmul,2\n#columns\n64,64,64,1,gfx950,half_tn_32x32x16,128,128,64,4,1\n")
    lc.tune_cache_load(str(p))
    lc.tune_cache_save(str(p))
    assert "64,64,64,1,gfx950,half_tn_32x32x16,128,128,64,4,1" in p.read_text()
    p.write_text("#lc_tune_cache,attention,9\n")
    with pytest.raises(RuntimeError, match="unsupported header"):
        lc.tune_cache_load(str(p))
