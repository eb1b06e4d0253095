"""matmul2d on the hip device vs the CPU oracle (src/ops/matmul_cpu.cpp:49-60).

Covers the reference's own cases (tests/test_matmul.cpp known answer,
tests/test_backend_parity.cpp 4x7x5 with atol 2e-3 / rtol 3e-3), the golden
vectors, BASELINE config 2 (fp32 1024^3 and 1000x1030x777) in full, config 5
(bf16 4096^3, 8192^3 on sampled rows plus a full-tensor column-checksum, and
the skinny 16x8192x8192 in full), the resident-session protocol and the
policy-level null-pointer contract.
"""
import numpy as np
import pytest

import oracle_lib
from gpu_util import assert_parity, note, require_hip
from lightning_core import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lc():
    return require_hip()


def test_matmul_kat(lc):
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(7, 13, dtype=np.float32).reshape(3, 2)
    out = lc.matmul2d(a, b)
    np.testing.assert_allclose(out, [[58, 64], [139, 154]], atol=1e-4)


@pytest.mark.parametrize("case", oracle_lib.golden_cases("matmul"), ids=lambda c: c["name"])
def test_matmul_golden(lc, case):
    p = case["params"]
    a = oracle_lib.golden_input(case, "a").reshape(p["m"], p["k"])
    b = oracle_lib.golden_input(case, "b").reshape(p["k"], p["n"])
    got = lc.matmul2d(a, b)
    exp = np.asarray(case["expected"], np.float32).reshape(p["m"], p["n"])
    assert_parity(exp, got, "f32", case["name"])
    assert oracle_lib.elementwise_ok(exp, got, 2e-3, 3e-3)


@pytest.mark.parametrize("m,k,n", [(1024, 1024, 1024), (1000, 777, 1030), (64, 64, 64), (1, 5, 300), (333, 17, 65)])
def test_matmul_f32_config2(lc, oracle, m, k, n):
    a = synth.uniform((m, k), stream=1)
    b = synth.uniform((k, n), stream=2)
    got = lc.matmul2d(a, b)
    assert_parity(oracle.matmul(a, b), got, "f32", f"f32 {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n", [(64, 8192, 64), (512, 4096, 512), (130, 1000, 70), (2048, 96, 2100), (65, 4500, 1),
                                   (700, 640, 900), (1000, 777, 1030)])
def test_matmul_f32_split_tiles(lc, oracle, m, k, n):
    # Shapes whose stream-K split puts one tile on several workgroups (up to
    # 128 partial tiles for 64x8192x64): the sum must match and be the same
    # bits on every run (partials are added in a fixed order).  512x4096x512,
    # 700x640x900 (165 tiles: XCD ranges of 20 and 21) and 1000x777x1030 take
    # the XCD-local split (fewer than two tiles per workgroup); 2048x96x2100
    # the global one.
    a = synth.uniform((m, k), stream=13)
    b = synth.uniform((k, n), stream=14)
    s = lc.MatMulResidentSession(m, k, n, "f32")
    s.start_into(a, b)
    first = s.finish_into().reshape(m, n).copy()
    s.run_batch_sync_cached_no_download(3)
    again = s.finish_into().reshape(m, n)
    assert_parity(oracle.matmul(a, b), first, "f32", f"f32 split {m}x{k}x{n}")
    np.testing.assert_array_equal(first, again)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("m,k,n", [(256, 320, 200), (300, 64, 520), (16, 512, 96), (7, 64, 1000), (1, 128, 33)])
def test_matmul_half_small(lc, oracle, dtype, m, k, n):
    a = synth.normal((m, k), stream=3)
    b = synth.normal((k, n), stream=4)
    s = lc.MatMulResidentSession(m, k, n, dtype)
    s.start_into(a, b)
    got = s.finish_into().reshape(m, n)
    ref = oracle.matmul(synth.round_to(a, dtype), synth.round_to(b, dtype))
    assert_parity(ref, got, dtype, f"{dtype} {m}x{k}x{n}")


def _colsum_check(a_r, b_r, got):
    # checksum of checksums: column sums of C equal (column sums of A) . B
    ref = np.asarray(a_r, np.float64).sum(axis=0) @ np.asarray(b_r, np.float64)
    err = oracle_lib.normwise_rel(ref, np.asarray(got, np.float64).sum(axis=0))
    note(f"[parity] colsum normwise_rel={err:.3e}")
    assert err <= 2e-3


@pytest.mark.parametrize("size", [4096, 8192])
def test_matmul_bf16_config5_sampled(lc, oracle, size):
    m = k = n = size
    note(f"[case] bf16 GEMM {size}^3 generating inputs")
    a = synth.normal((m, k), stream=5)
    b = synth.normal((k, n), stream=6)
    s = lc.MatMulResidentSession(m, k, n, "bf16")
    s.start_into(a, b)
    s.run_batch_sync_cached_no_download(3)
    got = s.finish_into().reshape(m, n)
    a_r, b_r = synth.round_bf16(a), synth.round_bf16(b)
    rows = np.unique(np.concatenate([np.arange(0, 32), np.linspace(32, m - 33, 16).astype(int), np.arange(m - 16, m)]))
    note(f"[case] oracle on {rows.size} sampled rows")
    for r0 in range(0, rows.size, 8):
        rr = rows[r0:r0 + 8]
        ref = np.concatenate([oracle.matmul(a_r, b_r, rows=(int(r), int(r) + 1)) for r in rr])
        assert_parity(ref, got[rr], "bf16", f"bf16 {size}^3 rows {rr[0]}..{rr[-1]}")
    _colsum_check(a_r, b_r, got)


def test_matmul_bf16_skinny_config5(lc, oracle):
    m, k, n = 16, 8192, 8192
    a = synth.normal((m, k), stream=7)
    b = synth.normal((k, n), stream=8)
    s = lc.MatMulResidentSession(m, k, n, "bf16")
    s.start_into(a, b)
    got = s.finish_into().reshape(m, n)
    ref = oracle.matmul(synth.round_bf16(a), synth.round_bf16(b))
    assert_parity(ref, got, "bf16", "bf16 skinny 16x8192x8192")


@pytest.mark.parametrize("m,k,n", [(16, 1000, 3000), (5, 960, 777), (16, 4096, 2048), (1, 2048, 130),
                                   (16, 320, 8192)])
def test_matmul_bf16_skinny_split_k(lc, oracle, m, k, n):
    """The skinny GEMM's split-K paths: ragged N (column tiles of 64) and K
    (a last k-block shorter than 256), M < 16, 1 to 8 splits.  Three
    launches on one session and a second session of the same shape must all
    match: the last workgroup of each column tile resets its counter, so a
    launch never sees another's counts."""
    a = synth.normal((m, k), stream=11)
    b = synth.normal((k, n), stream=12)
    ref = oracle.matmul(synth.round_bf16(a), synth.round_bf16(b))
    note(f"[case] skinny split-K {m}x{k}x{n}")
    s = lc.MatMulResidentSession(m, k, n, "bf16")
    s.start_into(a, b)
    first = s.finish_into().reshape(m, n).copy()
    assert_parity(ref, first, "bf16", f"bf16 skinny {m}x{k}x{n}")
    s2 = lc.MatMulResidentSession(m, k, n, "bf16")
    s2.start_into(a, b)
    s2.run_batch_sync_cached_no_download(3)
    again = s2.finish_into().reshape(m, n)
    # same partials, same k order: bit-identical
    np.testing.assert_array_equal(again, first)


@pytest.mark.parametrize("m,k,n", [(16, 4096, 8192), (7, 1000, 8200), (16, 8192, 8256)])
def test_matmul_bf16_skinny_unsplit(lc, oracle, m, k, n):
    """Column tiles for half the CUs or more: no split-K, each workgroup walks
    its k-blocks from block (5 * tile) mod nkb.  Ragged N (a last column tile
    past N) and K (a short last k-block that some workgroups read first);
    repeated launches are bit-identical."""
    a = synth.normal((m, k), stream=13)
    b = synth.normal((k, n), stream=14)
    note(f"[case] skinny unsplit {m}x{k}x{n}")
    s = lc.MatMulResidentSession(m, k, n, "bf16")
    s.start_into(a, b)
    first = s.finish_into().reshape(m, n).copy()
    a_r, b_r = synth.round_bf16(a), synth.round_bf16(b)
    cols = np.unique(np.concatenate([np.arange(0, 64), np.linspace(64, n - 65, 24).astype(int), np.arange(n - 64, n)]))
    ref = oracle.matmul(a_r, np.ascontiguousarray(b_r[:, cols]))
    assert_parity(ref, first[:, cols], "bf16", f"bf16 skinny unsplit {m}x{k}x{n}")
    s.run_batch_sync_cached_no_download(3)
    again = s.finish_into().reshape(m, n)
    np.testing.assert_array_equal(again, first)


def test_resident_session_protocol(lc, oracle):
    m, k, n = 96, 80, 72
    a = synth.uniform((m, k), stream=9)
    b = synth.uniform((k, n), stream=10)
    s = lc.MatMulResidentSession(m, k, n, "f32")
    out = s.start_into(a, b)  # no download: out untouched
    assert not out.any()
    s.run_into()
    s.sync_into()
    s.run_batch_sync_into(a, b, np.zeros(m * n, np.float32), 5)
    s.run_batch_sync_cached_no_download(4)
    got = s.finish_into().reshape(m, n)
    assert_parity(oracle.matmul(a, b), got, "f32", "resident protocol")
    # a second session of another shape does not disturb the first
    s2 = lc.MatMulResidentSession(8, 8, 8, "f32")
    s2.start_into(np.eye(8), np.eye(8))
    np.testing.assert_allclose(s2.finish_into().reshape(8, 8), np.eye(8))
    assert_parity(oracle.matmul(a, b), s.finish_into().reshape(m, n), "f32", "resident after other session")


def test_policy_null_pointers_use_resident(lc, oracle):
    m, k, n = 40, 30, 20
    a = synth.uniform((m, k), stream=11)
    b = synth.uniform((k, n), stream=12)
    start = lc.MatMulIoPolicy(upload_a=True, upload_b=True, download_out=False, synchronize=False)
    lc.matmul_with_policy(a, b, m, k, n, policy=start)
    run = lc.MatMulIoPolicy(upload_a=False, upload_b=False, download_out=True, synchronize=True)
    got = lc.matmul_with_policy(None, None, m, k, n, policy=run).reshape(m, n)
    assert_parity(oracle.matmul(a, b), got, "f32", "policy resident")
    # a null pointer that the policy needs is an invalid value (ops.hpp:367-370)
    with pytest.raises(RuntimeError, match="invalid value"):
        lc.matmul_with_policy(None, b, m, k, n, policy=lc.MatMulIoPolicy())


def test_plain_calls_in_a_row_and_resident_reuse(lc, oracle):
    """Plain fp32 calls (both operands uploaded, product downloaded) with at
    most 2^18 values per operand and product stage through pinned memory and
    wait on a completion flag raised by the kernel that copies the product
    out.  A run of them with changing shapes (across the size cap), mixed with
    plain attention calls that share the staging and the flag, each sees its
    own result, and the operands a plain call uploads stay resident."""
    shapes = [(1, 1, 1), (4, 7, 5), (64, 64, 64), (511, 512, 513), (512, 512, 512), (513, 512, 512),
              (3, 1000, 2), (200, 33, 1300)]
    for i, (m, k, n) in enumerate(shapes * 2):
        a = synth.uniform((m, k), stream=500 + 2 * i)
        b = synth.uniform((k, n), stream=501 + 2 * i)
        got = lc.matmul2d(a, b)
        assert_parity(oracle.matmul(a, b), got, "f32", f"call {i}: {m}x{k}x{n}")
        if i % 3 == 2:
            q, kk, v = (synth.normal((64, 32), stream=600 + 3 * i + j) for j in range(3))
            assert_parity(oracle.attention(q, kk, v), lc.attention2d(q, kk, v), "f32", f"attention {i}")
    m, k, n = 48, 40, 36
    a = synth.uniform((m, k), stream=590)
    b = synth.uniform((k, n), stream=591)
    first = lc.matmul_with_policy(a, b, m, k, n, policy=lc.MatMulIoPolicy()).reshape(m, n)
    run = lc.MatMulIoPolicy(upload_a=False, upload_b=False, download_out=True, synchronize=True)
    again = lc.matmul_with_policy(None, None, m, k, n, policy=run).reshape(m, n)
    exp = oracle.matmul(a, b)
    assert_parity(exp, first, "f32", "plain policy call")
    assert_parity(exp, again, "f32", "resident reuse after a plain call")


def test_matmul_f32_seeded_shape_sweep(lc, oracle):
    # 40 seeded fp32 shapes on both sides of the staging caps, as plain calls
    # and as a resident session's start / run / finish (small results come
    # back through the staged download), each against the oracle.
    rng = np.random.default_rng(20260402)
    for i in range(40):
        m, k, n = (int(x) for x in rng.integers(1, 700, size=3))
        a = synth.uniform((m, k), stream=1100 + 2 * i)
        b = synth.uniform((k, n), stream=1101 + 2 * i)
        ref = oracle.matmul(a, b)
        if i % 2 == 0:
            got = lc.matmul2d(a, b)
        else:
            s = lc.MatMulResidentSession(m, k, n, "f32")
            s.start_into(a, b)
            s.run_into()
            got = s.finish_into().reshape(m, n)
            s.close()
        assert_parity(ref, got, "f32", f"sweep {i}: {m}x{k}x{n}")


def test_trace_records_hip_dispatch(lc):
    lc.runtime_trace_clear()
    lc.runtime_trace_enable(True)
    try:
        lc.matmul2d(np.ones((4, 7), np.float32), np.ones((7, 5), np.float32))
    finally:
        lc.runtime_trace_enable(False)
    ev = [e for e in lc.runtime_trace_events() if e["type"] == "op_dispatch"]
    assert ev and ev[-1]["op"] == "matmul"
    assert ev[-1]["requested_device"] == "hip" and ev[-1]["selected_device"] == "hip" and not ev[-1]["fallback"]
    assert ev[-1]["size_bytes"] == 4 * 7 * 5


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_upload_rounding_bitexact(lc, dtype):
    # A . I with one nonzero per output sum is exact in fp32, so C equals the
    # device-rounded A bit for bit: the upload conversion must match the
    # round-to-nearest-even of lightning_core.synth (ties, tiny, large values).
    m, k = 16, 64
    rng = np.random.default_rng(5)
    base = rng.standard_normal((m, k)).astype(np.float32)
    bits = base.view(np.uint32)
    bits[0, :32] = (bits[0, :32] & 0xFFFF0000) | 0x8000  # exact bf16 ties
    bits[1, :32] = (bits[1, :32] & 0xFFFFE000) | 0x1000  # exact fp16 ties (normal range)
    base[2, :8] = [1e-30, -1e-30, 3e38, -3e38, 6e-5, 65504.0, 1e-8, 0.0]
    if dtype == "f16":
        base[2, 2:4] = [60000.0, -60000.0]
    s = lc.MatMulResidentSession(m, k, k, dtype)
    s.start_into(base, np.eye(k, dtype=np.float32))
    got = s.finish_into().reshape(m, k)
    exp = synth.round_to(base, dtype)
    # values, not bit patterns: a rounded -0.0 sums to +0.0 in the accumulator
    np.testing.assert_array_equal(got, exp)
