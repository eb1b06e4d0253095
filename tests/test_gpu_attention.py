"""attention2d on the hip device vs the CPU oracle (src/attention_cpu.cpp:38-101).

Covers the reference's known answer and postprocess closed form
(tests/test_attention.cpp:49-92), its parity case S=16 D=32 with
atol = rtol = 2e-2 (tests/test_backend_parity.cpp:158-185), the golden
vectors (odd shapes, causal), BASELINE config 1 (fp32 S=256 D=64) in full,
config 3 (bf16 causal B=4 H=16 S=2048 D=128) on sampled rows of every head
plus two heads in full plus the convex-hull property on the whole tensor,
fp16, and the session upload-once protocol.
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


def test_attention_kat_and_postprocess(lc):
    eye = np.eye(2, dtype=np.float32)
    v = np.diag([10.0, 20.0]).astype(np.float32)
    out = lc.attention2d(eye, eye, v)
    np.testing.assert_allclose(out, [[6.6976, 6.6048], [3.3024, 13.3952]], atol=0.05)
    a = np.exp(1 / np.sqrt(2)) / (1 + np.exp(1 / np.sqrt(2)))
    exact = np.array([[10 * a, 20 * (1 - a)], [10 * (1 - a), 20 * a]])
    np.testing.assert_allclose(out, exact, rtol=1e-5)
    post = lc.AttentionIoPolicy(output_scale=0.5, output_bias=-2.0, output_relu=True)
    got = lc.attention_forward_with_policy(eye, eye, v, 2, 2, policy=post).reshape(2, 2)
    np.testing.assert_allclose(got, np.maximum(exact * 0.5 - 2.0, 0), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("case", oracle_lib.golden_cases("attention"), ids=lambda c: c["name"])
def test_attention_golden(lc, case):
    p = case["params"]
    s, d = p["seq_len"], p["head_dim"]
    q, k, v = (oracle_lib.golden_input(case, n).reshape(s, d) for n in "qkv")
    pol = lc.AttentionIoPolicy(output_scale=p["output_scale"], output_bias=p["output_bias"],
                               output_relu=p["output_relu"])
    got = lc.attention_forward_with_policy(q, k, v, s, d, p["causal"], policy=pol)
    exp = np.asarray(case["expected"], np.float32)
    assert_parity(exp, got, "f32", case["name"])
    assert oracle_lib.elementwise_ok(exp, got, 2e-2, 2e-2)


@pytest.mark.parametrize("s,d,causal", [(256, 64, False), (256, 64, True), (100, 96, True), (31, 200, False),
                                        (1, 8, False), (513, 128, True)])
def test_attention_f32(lc, oracle, s, d, causal):
    q, k, v = (synth.normal((s, d), stream=i) for i in range(3))
    got = lc.attention2d(q, k, v, causal)
    assert_parity(oracle.attention(q, k, v, causal), got, "f32", f"f32 S={s} D={d} causal={causal}")


@pytest.mark.parametrize("s,d,causal", [(2048, 64, True), (1024, 128, False), (700, 200, True), (256, 256, False),
                                        (33, 256, True), (1100, 36, False)])
def test_attention_f32_key_split(lc, oracle, s, d, causal):
    # Grids of fewer than 128 query blocks divide each block's keys among up
    # to 16 workgroups (a causal block's later splits can be empty: S=33);
    # a second kernel merges the partials in split order, so repeated calls
    # give the same bits.
    q, k, v = (synth.normal((s, d), stream=800 + i) for i in range(3))
    got = lc.attention2d(q, k, v, causal)
    assert_parity(oracle.attention(q, k, v, causal), got, "f32", f"f32 key split S={s} D={d} causal={causal}")
    np.testing.assert_array_equal(lc.attention2d(q, k, v, causal), got)


def test_attention_f32_seeded_shape_sweep(lc, oracle):
    # 40 seeded shapes across the kernel choices (16-query kernel, 32-query
    # kernel with and without key splits, float4 and scalar tile fills,
    # plain-call staging and pageable copies), causal or not, with and
    # without the output postprocess, each against the oracle.
    rng = np.random.default_rng(20260401)
    done = 0
    while done < 40:
        s = int(rng.integers(1, 2200))
        d = int(rng.choice([1, 3, 4, 8, 16, 31, 32, 48, 64, 65, 96, 128, 160, 200, 255, 256]))
        if s * s * d > 3e8:
            continue
        causal = bool(rng.integers(0, 2))
        q, k, v = (synth.normal((s, d), stream=1000 + 3 * done + j) for j in range(3))
        ref = oracle.attention(q, k, v, causal)
        if rng.integers(0, 3) == 0:
            pol = lc.AttentionIoPolicy(output_scale=1.5, output_bias=-0.25, output_relu=True)
            got = lc.attention_forward_with_policy(q, k, v, s, d, causal, policy=pol).reshape(s, d)
            ref = np.maximum(ref * 1.5 - 0.25, 0)
        else:
            got = lc.attention2d(q, k, v, causal)
        assert_parity(ref, got, "f32", f"sweep {done}: S={s} D={d} causal={causal}")
        done += 1


def test_attention_f32_batched_key_split(lc, oracle):
    b, h, s, d = 1, 3, 300, 128
    q, k, v = (synth.normal((b, h, s, d), stream=820 + i) for i in range(3))
    got = lc.attention_batched(q, k, v, True, "f32")
    for hi in range(h):
        assert_parity(oracle.attention(q[0, hi], k[0, hi], v[0, hi], True), got[0, hi], "f32", f"f32 batched head {hi}")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("b,h,s,d,causal", [(1, 2, 70, 64, True), (2, 3, 196, 64, False), (1, 2, 33, 128, True),
                                            (1, 1, 300, 128, False), (2, 2, 128, 64, True)])
def test_attention_half_small(lc, oracle, dtype, b, h, s, d, causal):
    shape = (b, h, s, d)
    q, k, v = (0.5 * synth.normal(shape, stream=10 + i) for i in range(3))
    got = lc.attention_batched(q, k, v, causal, dtype)
    ref = oracle.attention_batched(*(synth.round_to(x, dtype) for x in (q, k, v)), causal)
    assert_parity(ref, got, dtype, f"{dtype} {shape} causal={causal}")


def test_attention_bf16_config3(lc, oracle):
    b, h, s, d = 4, 16, 2048, 128
    shape = (b, h, s, d)
    note("[case] config 3 generating inputs")
    q, k, v = (0.5 * synth.normal(shape, stream=20 + i) for i in range(3))
    sess = lc.AttentionSession.batched(b, h, s, d, causal=True, compute_dtype="bf16")
    out = np.zeros(q.size, np.float32)
    sess.forward_with_policy_into(q, k, v, out, lc.AttentionIoPolicy())
    sess.run_cached(2)
    got = out.reshape(shape)
    qr, kr, vr = (synth.round_bf16(x) for x in (q, k, v))
    rows = (0, 1, 63, 64, 127, 128, 1000, 2046, 2047)
    note("[case] oracle on sampled rows of all 64 heads")
    for r in rows:
        ref = oracle.attention_batched_rows(qr, kr, vr, True, (r, r + 1))
        assert_parity(ref, got[:, :, r:r + 1, :], "bf16", f"config3 row {r}")
    for bi, hi in ((0, 0), (3, 15)):
        ref = oracle.attention(qr[bi, hi], kr[bi, hi], vr[bi, hi], True)
        assert_parity(ref, got[bi, hi], "bf16", f"config3 head ({bi},{hi}) full")
    # every output row is a convex combination of the visible V rows
    vmin = np.minimum.accumulate(vr, axis=2)
    vmax = np.maximum.accumulate(vr, axis=2)
    slack = 1e-2 * np.abs(vr).max()
    assert np.all(got >= vmin - slack) and np.all(got <= vmax + slack)


def test_session_upload_once(lc, oracle):
    s, d = 64, 32
    q, k, v = (synth.normal((s, d), stream=40 + i) for i in range(3))
    sess = lc.AttentionSession(s, d, causal=False)
    pol = sess.default_policy()
    assert not pol.synchronize  # session default (reference src/attention.cpp:249-253)
    sess.forward_with_policy(q, k, v, lc.AttentionIoPolicy(download_out=False))
    # reuse resident q/k/v: host arguments are ignored when not uploaded
    junk = np.full((s, d), np.nan, np.float32)
    got = sess.forward_with_policy(junk, junk, junk, lc.AttentionIoPolicy(upload_q=False, upload_k=False,
                                                                          upload_v=False))
    assert_parity(oracle.attention(q, k, v), got.reshape(s, d), "f32", "session resident")
    # new k only
    k2 = synth.normal((s, d), stream=44)
    got = sess.forward_with_policy(junk, k2, junk, lc.AttentionIoPolicy(upload_q=False, upload_v=False))
    assert_parity(oracle.attention(q, k2, v), got.reshape(s, d), "f32", "session partial upload")
    fresh = lc.AttentionSession(s, d)
    with pytest.raises(RuntimeError, match="invalid value"):
        fresh.forward_with_policy(q, k, v, lc.AttentionIoPolicy(upload_q=False))


def test_plain_calls_in_a_row_and_resident_reuse(lc, oracle):
    """Plain calls (every input uploaded, output downloaded) of one head up to
    65536 values per tensor stage through pinned memory and wait on a
    completion flag; a run of them with changing shapes, causal and
    postprocess settings, interleaved with the fused conv -> attention call
    (which shares the staging and the flag), each sees its own result, and
    the inputs a plain session call uploads stay resident for later calls."""
    shapes = [(64, 32), (256, 64), (17, 5), (128, 256), (1, 8), (64, 32), (256, 256), (300, 200)]
    x = synth.normal((1, 3, 8, 8), stream=330)
    w = synth.normal((16, 3, 3, 3), stream=331)
    for i, (s, d) in enumerate(shapes * 2):
        q, k, v = (synth.normal((s, d), stream=340 + 3 * i + j) for j in range(3))
        causal = i % 3 == 1
        if i % 4 == 2:
            pol = lc.AttentionIoPolicy(output_scale=0.5, output_bias=-0.1, output_relu=True)
            got = lc.attention_forward_with_policy(q, k, v, s, d, causal, policy=pol).reshape(s, d)
            exp = np.maximum(oracle.attention(q, k, v, causal) * 0.5 - 0.1, 0)
        else:
            got = lc.attention2d(q, k, v, causal)
            exp = oracle.attention(q, k, v, causal)
        assert_parity(exp, got, "f32", f"call {i}: S={s} D={d} causal={causal}")
        if i % 5 == 4:
            ca = lc.api.conv_attention_torchstrong_nchw(x, w, None, 48, 48, 1, 1, 1, 1)
            ref = oracle.conv_attention(x, w, None, 48, 48, (1, 1), (1, 1))
            assert_parity(ref.ravel(), np.asarray(ca).ravel(), "f32", f"conv {i}")
    s, d = 256, 64
    q, k, v = (synth.normal((s, d), stream=390 + j) for j in range(3))
    sess = lc.AttentionSession(s, d, causal=True)
    first = sess.forward_with_policy(q, k, v, lc.AttentionIoPolicy())
    junk = np.full((s, d), np.nan, np.float32)
    again = sess.forward_with_policy(junk, junk, junk, lc.AttentionIoPolicy(upload_q=False, upload_k=False,
                                                                            upload_v=False))
    exp = oracle.attention(q, k, v, True)
    assert_parity(exp, first.reshape(s, d), "f32", "plain session call")
    assert_parity(exp, again.reshape(s, d), "f32", "resident reuse after a plain call")


def test_attention_trace(lc):
    lc.runtime_trace_clear()
    lc.runtime_trace_enable(True)
    try:
        lc.attention2d(np.eye(4, 8, dtype=np.float32), np.eye(4, 8, dtype=np.float32), np.ones((4, 8), np.float32))
    finally:
        lc.runtime_trace_enable(False)
    ev = [e for e in lc.runtime_trace_events() if e["type"] == "op_dispatch"]
    assert ev[-1]["op"] == "attention_forward" and ev[-1]["selected_device"] == "hip"
    assert ev[-1]["size_bytes"] == 4 * 4 * 8
