"""lcMatMulDeviceNoAlloc, the fp32 GEMM entry point that allocates nothing,
against lcMatMul (the entry point whose kernels it shares) and the CPU oracle.

Device buffers come from lcMalloc once, before the calls under test.  Two
calls in a row, the second with a smaller input (the shared scratch keeps the
first call's contents: stale partial tiles, flags of an earlier epoch); each
result is checked against lcMatMul's on the same inputs and against the
oracle, to the fp32 bar (normwise 1e-4).  Shapes cover whole tiles, stream-K
split tiles, padded operands (dims not multiples of 64) and a misaligned
base; a shape whose padded copies exceed the scratch is refused.  The
defining property is checked directly too: after one warm-up call (module
load, the symbol's address), free device memory as HIP reports it does not
move across calls that pad, misalign and split tiles with stream-K.
"""
import ctypes

import numpy as np
import pytest

from gpu_util import assert_parity, note, require_hip
from lightning_core import _native as N
from lightning_core import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lc():
    return require_hip()


class DeviceArrays:
    """lcMalloc'd device buffers, freed at the end."""

    def __init__(self, lib):
        self.lib = lib
        self.ptrs = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.lib.lcMalloc(ctypes.byref(p), nbytes) == N.LC_SUCCESS
        self.ptrs.append(p)
        return p.value

    def close(self):
        for p in self.ptrs:
            self.lib.lcFree(p)


def _upload(lib, dptr, host):
    host = np.ascontiguousarray(host, np.float32)
    assert lib.lcMemcpy(ctypes.c_void_p(dptr), host.ctypes.data_as(ctypes.c_void_p), host.nbytes,
                        N.LC_MEMCPY_HOST_TO_DEVICE) == N.LC_SUCCESS


def _download(lib, dptr, shape):
    out = np.empty(shape, np.float32)
    assert lib.lcMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(dptr), out.nbytes,
                        N.LC_MEMCPY_DEVICE_TO_HOST) == N.LC_SUCCESS
    return out


# (first call, second smaller call); the byte offset shifts A off 16-byte alignment
PAIRS = [((1024, 1024, 1024), (256, 512, 128)),      # whole tiles, no padded copies
         ((1000, 777, 1030), (300, 129, 200)),       # stream-K split tiles + padded copies
         ((512, 4096, 512), (64, 8192, 64)),         # long K: many partial tiles per output tile
         ((640, 640, 640), (129, 64, 65))]


@pytest.mark.parametrize("first,second", PAIRS, ids=lambda s: "x".join(map(str, s)))
def test_no_alloc_matches_lcmatmul(lc, oracle, first, second):
    lib = N.load()
    dev = DeviceArrays(lib)
    try:
        mx, kx, nx = (max(a, b) for a, b in zip(first, second))
        da = dev.alloc(mx * kx * 4 + 16)
        db = dev.alloc(kx * nx * 4)
        dc = dev.alloc(mx * nx * 4)
        for i, (m, k, n) in enumerate((first, second)):
            note(f"[case] no-alloc {m}x{k}x{n} (call {i + 1} of 2)")
            a = synth.uniform((m, k), stream=300 + 2 * i)
            b = synth.uniform((k, n), stream=301 + 2 * i)
            _upload(lib, da, a)
            _upload(lib, db, b)
            st = lib.lcMatMulDeviceNoAlloc(ctypes.c_void_p(da), ctypes.c_void_p(db), ctypes.c_void_p(dc), m, k, n)
            assert st == N.LC_SUCCESS, lib.lcGetLastErrorMessage().decode()
            got = _download(lib, dc, (m, n))
            ref_entry = lc.matmul2d(a, b)
            assert_parity(ref_entry, got, "f32", f"no-alloc vs lcMatMul {m}x{k}x{n}")
            assert_parity(oracle.matmul(a, b), got, "f32", f"no-alloc vs oracle {m}x{k}x{n}")
        # misaligned A base (4 bytes past the allocation): copied into the scratch
        m, k, n = second
        a = synth.uniform((m, k), stream=310)
        b = synth.uniform((k, n), stream=311)
        _upload(lib, da + 4, a)
        _upload(lib, db, b)
        st = lib.lcMatMulDeviceNoAlloc(ctypes.c_void_p(da + 4), ctypes.c_void_p(db), ctypes.c_void_p(dc), m, k, n)
        assert st == N.LC_SUCCESS, lib.lcGetLastErrorMessage().decode()
        assert_parity(oracle.matmul(a, b), _download(lib, dc, (m, n)), "f32", f"no-alloc misaligned A {m}x{k}x{n}")
    finally:
        dev.close()


def test_no_alloc_refuses_what_it_cannot_hold(lc):
    lib = N.load()
    dev = DeviceArrays(lib)
    try:
        d = dev.alloc(4096)
        # 3000 x 3001 x 3000: padded copies of ~74 MB, beyond the fixed scratch (checked before any launch)
        st = lib.lcMatMulDeviceNoAlloc(ctypes.c_void_p(d), ctypes.c_void_p(d), ctypes.c_void_p(d), 3000, 3001, 3000)
        assert st == N.LC_NOT_SUPPORTED
        assert "scratch" in lib.lcGetLastErrorMessage().decode()
        # host memory is not device memory
        host = np.zeros(64 * 64, np.float32)
        hp = host.ctypes.data_as(ctypes.c_void_p)
        assert lib.lcMatMulDeviceNoAlloc(hp, ctypes.c_void_p(d), ctypes.c_void_p(d), 8, 8, 8) == N.LC_INVALID_VALUE
        assert lib.lcMatMulDeviceNoAlloc(None, ctypes.c_void_p(d), ctypes.c_void_p(d), 8, 8, 8) == N.LC_INVALID_VALUE
        assert lib.lcMatMulDeviceNoAlloc(ctypes.c_void_p(d), ctypes.c_void_p(d), ctypes.c_void_p(d), 0, 8, 8) == \
            N.LC_INVALID_VALUE
    finally:
        dev.close()


def _free_device_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_no_alloc_allocates_nothing(lc, oracle):
    lib = N.load()
    dev = DeviceArrays(lib)
    shapes = [(1000, 777, 1030),   # stream-K split tiles + padded copies of A and B
              (512, 4096, 512),    # long K, whole tiles, no copies
              (129, 64, 65)]       # padded copies of a small shape
    try:
        da = dev.alloc(1024 * 4096 * 4 + 16)
        db = dev.alloc(4096 * 1030 * 4)
        dc = dev.alloc(1024 * 1030 * 4)
        inputs = []
        for i, (m, k, n) in enumerate(shapes):
            inputs.append((synth.uniform((m, k), stream=320 + 2 * i), synth.uniform((k, n), stream=321 + 2 * i)))
        # warm-up: loads the module and takes the scratch symbol's address
        a0, b0 = inputs[0]
        _upload(lib, da, a0)
        _upload(lib, db, b0)
        m, k, n = shapes[0]
        assert lib.lcMatMulDeviceNoAlloc(ctypes.c_void_p(da), ctypes.c_void_p(db), ctypes.c_void_p(dc),
                                         m, k, n) == N.LC_SUCCESS
        assert lib.lcDeviceSynchronize() == N.LC_SUCCESS
        before = _free_device_bytes()
        results = []
        for (m, k, n), (a, b) in zip(shapes, inputs):
            for off in (0, 4):  # aligned, then a base 4 bytes off (copied into the scratch)
                note(f"[case] no-alloc memory check {m}x{k}x{n} offset {off}")
                _upload(lib, da + off, a)
                _upload(lib, db, b)
                st = lib.lcMatMulDeviceNoAlloc(ctypes.c_void_p(da + off), ctypes.c_void_p(db),
                                               ctypes.c_void_p(dc), m, k, n)
                assert st == N.LC_SUCCESS, lib.lcGetLastErrorMessage().decode()
                results.append(((m, k, n), off, _download(lib, dc, (m, n))))
        after = _free_device_bytes()
        assert after == before, f"free device memory moved by {before - after} bytes"
        for (m, k, n), off, got in results:
            a, b = inputs[shapes.index((m, k, n))]
            assert_parity(oracle.matmul(a, b), got, "f32", f"no-alloc {m}x{k}x{n} offset {off}")
    finally:
        dev.close()
