"""Pins the CPU oracle before anything is checked against it (CPU only).

Each oracle function is checked against (a) the golden vectors written from the
reference's own compiled CPU path (tests/golden), (b) the reference's
known-answer tests, and (c) what the mathematics fixes: float64 brute force,
softmax invariants, direct convolution, numpy tiling.  The sensitivity tests at
the end plant mistakes in the oracle's inputs and show the checks catch them.
"""
import numpy as np
import pytest

import oracle_lib
from lightning_core import synth

GOLD_TOL = 2e-6  # oracle vs compiled reference: same algorithm, same flags


def _bf_attention(q, k, v, causal):
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    s, d = q.shape
    sc = q @ k.T / np.sqrt(d)
    if causal:
        sc = np.where(np.triu(np.ones((s, s), bool), 1), -np.inf, sc)
    sc -= sc.max(axis=1, keepdims=True)
    p = np.exp(sc)
    p /= p.sum(axis=1, keepdims=True)
    return p @ v


def _direct_conv(x, w, bias, stride, pad, relu):
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    bn, c, h, wd = x.shape
    oc, _, kh, kw = w.shape
    xp = np.zeros((bn, c, h + 2 * pad[0], wd + 2 * pad[1]))
    xp[:, :, pad[0]:pad[0] + h, pad[1]:pad[1] + wd] = x
    oh = (h + 2 * pad[0] - kh) // stride[0] + 1
    ow = (wd + 2 * pad[1] - kw) // stride[1] + 1
    out = np.zeros((bn, oc, oh, ow))
    for oy in range(oh):
        for ox in range(ow):
            patch = xp[:, :, oy * stride[0]:oy * stride[0] + kh, ox * stride[1]:ox * stride[1] + kw]
            out[:, :, oy, ox] = np.einsum("bckl,ockl->bo", patch, w)
    if bias is not None:
        out += np.asarray(bias, np.float64)[None, :, None, None]
    return np.maximum(out, 0) if relu else out


# --- (a) golden vectors from the compiled reference ---------------------------

@pytest.mark.parametrize("case", oracle_lib.golden_cases("attention"), ids=lambda c: c["name"])
def test_attention_golden(oracle, case):
    p = case["params"]
    s, d = p["seq_len"], p["head_dim"]
    q, k, v = (oracle_lib.golden_input(case, n).reshape(s, d) for n in "qkv")
    out = oracle.attention(q, k, v, p["causal"])
    out = oracle.postprocess(out, p["output_scale"], p["output_bias"], p["output_relu"])
    assert oracle_lib.normwise_rel(case["expected"], out.ravel()) <= GOLD_TOL


@pytest.mark.parametrize("case", oracle_lib.golden_cases("matmul"), ids=lambda c: c["name"])
def test_matmul_golden(oracle, case):
    p = case["params"]
    a = oracle_lib.golden_input(case, "a").reshape(p["m"], p["k"])
    b = oracle_lib.golden_input(case, "b").reshape(p["k"], p["n"])
    assert oracle_lib.normwise_rel(case["expected"], oracle.matmul(a, b).ravel()) <= GOLD_TOL


@pytest.mark.parametrize("case", oracle_lib.golden_cases("conv_"), ids=lambda c: c["name"])
def test_conv_golden(oracle, case):
    p = case["params"]
    x = oracle_lib.golden_input(case, "x").reshape(p["batch"], p["in_c"], p["in_h"], p["in_w"])
    w = oracle_lib.golden_input(case, "w").reshape(p["out_c"], p["in_c"], p["kh"], p["kw"])
    bias = oracle_lib.golden_input(case, "bias")
    stride, pad = (p["stride_h"], p["stride_w"]), (p["pad_h"], p["pad_w"])
    if p["op"] == "conv2d_nchw":
        got = oracle.conv2d(x, w, bias, stride, pad, p["relu"])
    else:
        got = oracle.conv_attention(x, w, bias, p["seq_len"], p["head_dim"], stride, pad)
    assert oracle_lib.normwise_rel(case["expected"], got.ravel()) <= GOLD_TOL


# --- (b) the reference's known-answer tests -----------------------------------

def test_attention_kat(oracle):
    # tests/test_attention.cpp:49-68; closed form e^{1/sqrt2}/(1+e^{1/sqrt2}).
    eye = np.eye(2, dtype=np.float32)
    v = np.diag([10.0, 20.0]).astype(np.float32)
    out = oracle.attention(eye, eye, v)
    a = np.exp(1 / np.sqrt(2)) / (1 + np.exp(1 / np.sqrt(2)))
    exact = np.array([[10 * a, 20 * (1 - a)], [10 * (1 - a), 20 * a]])
    np.testing.assert_allclose(out, [[6.6976, 6.6048], [3.3024, 13.3952]], atol=0.05)
    np.testing.assert_allclose(out, exact, rtol=1e-5)
    # tests/test_attention.cpp:70-92: postprocess closed form.
    post = oracle.postprocess(out, 0.5, -2.0, True)
    np.testing.assert_allclose(post, np.maximum(exact * 0.5 - 2.0, 0), rtol=1e-5, atol=1e-6)


def test_postprocess_identity_and_relu(oracle):
    x = synth.normal((50,), seed=3)
    np.testing.assert_array_equal(oracle.postprocess(x, 1.0, 0.0, False), x)
    np.testing.assert_allclose(oracle.postprocess(x, 2.0, 0.5, False), 2 * x + 0.5, rtol=1e-6)
    assert np.all(oracle.postprocess(x, 1.0, 0.0, True) >= 0)


def test_matmul_kat(oracle):
    # tests/test_matmul.cpp:14-50.
    a = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    b = np.arange(7, 13, dtype=np.float32).reshape(3, 2)
    np.testing.assert_array_equal(oracle.matmul(a, b), [[58, 64], [139, 154]])


# --- (c) mathematics ------------------------------------------------------------

@pytest.mark.parametrize("s,d,causal", [(1, 1, False), (7, 5, True), (31, 17, False), (48, 64, True)])
def test_attention_bruteforce(oracle, s, d, causal):
    q, k, v = (synth.normal((s, d), seed=21, stream=i) for i in range(3))
    got = oracle.attention(q, k, v, causal)
    assert oracle_lib.normwise_rel(_bf_attention(q, k, v, causal), got) < 1e-5


def test_attention_invariants(oracle):
    s, d = 40, 24
    q, k = synth.normal((s, d), seed=9, stream=1), synth.normal((s, d), seed=9, stream=2)
    # constant V rows -> every output row equals that row (softmax rows sum to 1)
    row = synth.normal((d,), seed=9, stream=3)
    out = oracle.attention(q, k, np.tile(row, (s, 1)))
    np.testing.assert_allclose(out, np.tile(row, (s, 1)), rtol=1e-5, atol=1e-6)
    # causal row 0 sees only key 0 -> out[0] = V[0]
    v = synth.normal((s, d), seed=9, stream=4)
    out = oracle.attention(q, k, v, causal=True)
    np.testing.assert_allclose(out[0], v[0], rtol=1e-6)
    # causal row i equals non-causal attention over the prefix 0..i
    i = 17
    pre = oracle.attention(q[: i + 1], k[: i + 1], v[: i + 1])
    np.testing.assert_allclose(out[i], pre[i], rtol=1e-5, atol=1e-6)
    # q = 0 -> uniform weights -> column mean of V
    out = oracle.attention(np.zeros((s, d), np.float32), k, v)
    np.testing.assert_allclose(out, np.tile(v.mean(axis=0), (s, 1)), rtol=1e-4, atol=1e-5)


def _batched_with_head_stride(oracle, q, k, v, causal, stride):
    """The batched loop rebuilt from the per-head C function with an explicit
    head stride (floats): the correct stride is S*D; other strides plant an
    indexing mistake for the sensitivity check below."""
    import ctypes

    b, h, s, d = q.shape
    q, k, v = (np.ascontiguousarray(x, np.float32) for x in (q, k, v))
    out = np.zeros_like(q)
    base = [x.ctypes.data for x in (q, k, v, out)]
    for bh in range(b * h):
        off = 4 * bh * stride
        st = oracle.lib.orc_attention_forward(*(ctypes.c_void_p(p + off) for p in base), s, d, int(causal))
        assert st == 0
    return out


@pytest.mark.parametrize("shape,causal", [((2, 3, 19, 8), False), ((2, 3, 19, 8), True), ((1, 4, 40, 24), True),
                                          ((3, 1, 1, 5), False)])
def test_attention_batched_pinned(oracle, shape, causal):
    """orc_attention_forward_batched (the checker of every batched GPU case):
    bit-equal to the per-head function on each [S, D] slice, and within 1e-5
    of float64 brute force per head."""
    q, k, v = (synth.normal(shape, seed=41, stream=i) for i in range(3))
    got = oracle.attention_batched(q, k, v, causal)
    b, h, s, d = shape
    for bi in range(b):
        for hi in range(h):
            np.testing.assert_array_equal(got[bi, hi], oracle.attention(q[bi, hi], k[bi, hi], v[bi, hi], causal))
            ref = _bf_attention(q[bi, hi], k[bi, hi], v[bi, hi], causal)
            assert oracle_lib.normwise_rel(ref, got[bi, hi]) < 1e-5
    np.testing.assert_array_equal(got, _batched_with_head_stride(oracle, q, k, v, causal, s * d))


def test_attention_batched_catches_stride_mistake(oracle):
    """A head offset of bh*S instead of bh*S*D (a dropped factor) fails the
    per-head brute-force check the batched pin uses."""
    shape = (2, 3, 16, 8)
    q, k, v = (synth.normal(shape, seed=42, stream=i) for i in range(3))
    s, d = shape[2], shape[3]
    wrong = _batched_with_head_stride(oracle, q, k, v, True, s)
    errs = [oracle_lib.normwise_rel(_bf_attention(q[bi, hi], k[bi, hi], v[bi, hi], True), wrong[bi, hi])
            for bi in range(2) for hi in range(3)]
    assert max(errs) > 1e-2


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (33, 64, 17)])
def test_matmul_bruteforce(oracle, m, k, n):
    a, b = synth.uniform((m, k), seed=4, stream=1), synth.uniform((k, n), seed=4, stream=2)
    ref = np.asarray(a, np.float64) @ np.asarray(b, np.float64)
    assert oracle_lib.normwise_rel(ref, oracle.matmul(a, b)) < 1e-6


def test_row_subsets_match_full(oracle):
    q, k, v = (synth.normal((37, 16), seed=2, stream=i) for i in range(3))
    full = oracle.attention(q, k, v, True)
    np.testing.assert_array_equal(oracle.attention(q, k, v, True, rows=(5, 23)), full[5:23])
    a, b = synth.uniform((29, 13), seed=2, stream=5), synth.uniform((13, 11), seed=2, stream=6)
    np.testing.assert_array_equal(oracle.matmul(a, b, rows=(3, 20)), oracle.matmul(a, b)[3:20])


@pytest.mark.parametrize("dims", [((2, 3, 8, 8), (4, 3, 3, 3), (1, 1), (1, 1)),
                                  ((1, 2, 9, 7), (5, 2, 3, 2), (2, 1), (1, 0)),
                                  ((2, 3, 32, 32), (6, 3, 16, 16), (16, 16), (0, 0))])
def test_conv_direct(oracle, dims):
    xs, ws, stride, pad = dims
    x, w = synth.normal(xs, seed=8, stream=1), synth.normal(ws, seed=8, stream=2)
    bias = synth.normal((ws[0],), seed=8, stream=3)
    for relu in (False, True):
        got = oracle.conv2d(x, w, bias, stride, pad, relu)
        assert oracle_lib.normwise_rel(_direct_conv(x, w, bias, stride, pad, relu), got) < 1e-5


@pytest.mark.parametrize("conv_size,need", [(10, 4), (7, 20), (30, 10), (5, 5), (1, 3)])
def test_qkv_pack_repeat_closed_form(oracle, conv_size, need):
    conv = synth.normal((conv_size,), seed=1)
    got = oracle.qkv_pack_repeat(conv, need)
    np.testing.assert_array_equal(got, np.resize(conv, 3 * need))


def _vit_numpy(x, w_conv, w_qkv, w_o, heads):
    x = np.asarray(x, np.float64)
    bn, c, h, w = x.shape
    e, _, p, _ = w_conv.shape
    g_h, g_w = h // p, w // p
    patches = x.reshape(bn, c, g_h, p, g_w, p).transpose(0, 2, 4, 1, 3, 5).reshape(bn, g_h * g_w, c * p * p)
    tok = np.maximum(patches @ np.asarray(w_conv, np.float64).reshape(e, -1).T, 0)
    t = g_h * g_w
    dh = e // heads
    qkv = (tok @ np.asarray(w_qkv, np.float64)).reshape(bn, t, 3, heads, dh).transpose(2, 0, 3, 1, 4)
    q, k, v = qkv[0], qkv[1], qkv[2]
    sc = q @ k.transpose(0, 1, 3, 2) / np.sqrt(dh)
    sc -= sc.max(-1, keepdims=True)
    pr = np.exp(sc)
    pr /= pr.sum(-1, keepdims=True)
    o = (pr @ v).transpose(0, 2, 1, 3).reshape(bn, t, e)
    return (o @ np.asarray(w_o, np.float64)).reshape(bn * t, e)


def test_vit_block_composition(oracle):
    bn, c, img, p, e, heads = 2, 3, 32, 8, 48, 4
    x = synth.uniform((bn, c, img, img), seed=12, lo=0, hi=1, stream=1)
    w_conv = synth.normal((e, c, p, p), seed=12, std=0.02, stream=2)
    w_qkv = synth.normal((e, 3 * e), seed=12, std=0.02, stream=3)
    w_o = synth.normal((e, e), seed=12, std=0.02, stream=4)
    ref = _vit_numpy(x, w_conv, w_qkv, w_o, heads)
    got = oracle.vit_block(x, w_conv, w_qkv, w_o, heads)
    assert oracle_lib.normwise_rel(ref, got) < 1e-5
    np.testing.assert_array_equal(oracle.vit_block(x, w_conv, w_qkv, w_o, heads, rows=(10, 30)), got[10:30])


# --- attention train step (src/attention_cpu.cpp:114-163) -----------------------

def _bf_train_step(q, k, v, t, lr, causal):
    """float64: forward, mean squared error, grad_v = P^T . 2(out - t)/(S*D), SGD."""
    q, k, v, t = (np.asarray(x, np.float64) for x in (q, k, v, t))
    s, d = q.shape
    sc = q @ k.T / np.sqrt(d)
    if causal:
        sc = np.where(np.triu(np.ones((s, s), bool), 1), -np.inf, sc)
    p = np.exp(sc - sc.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    out = p @ v
    go = 2.0 * (out - t) / (s * d)
    return out, v - lr * (p.T @ go), float(np.mean((out - t) ** 2))


@pytest.mark.parametrize("case", oracle_lib.golden_cases("train_attention"), ids=lambda c: c["name"])
def test_train_step_golden(oracle, case):
    p = case["params"]
    s, d = p["seq_len"], p["head_dim"]
    q, k, v, t = (oracle_lib.golden_input(case, n).reshape(s, d) for n in ("q", "k", "v", "target"))
    out, v_new, loss = oracle.attention_train_step(q, k, v, t, p["learning_rate"], p["causal"])
    exp = np.asarray(case["expected"], np.float32)
    assert oracle_lib.normwise_rel(exp[:s * d], out.ravel()) <= GOLD_TOL
    assert oracle_lib.normwise_rel(exp[s * d:2 * s * d], v_new.ravel()) <= GOLD_TOL
    assert abs(loss - exp[-1]) <= GOLD_TOL * abs(exp[-1])


@pytest.mark.parametrize("s,d,causal,lr", [(17, 8, False, 5.0), (40, 33, True, 20.0), (64, 64, True, 50.0)])
def test_train_step_bruteforce(oracle, s, d, causal, lr):
    # learning rates large enough that the update (~lr * 2|out - t| / (S*D))
    # dwarfs the fp32 rounding of v itself, so the update is checked on its own
    q, k, v, t = (synth.normal((s, d), seed=40, stream=i) for i in range(4))
    out, v_new, loss = oracle.attention_train_step(q, k, v, t, lr, causal)
    bo, bv, bl = _bf_train_step(q, k, v, t, lr, causal)
    assert oracle_lib.normwise_rel(bo, out) <= 1e-5
    upd = bv - np.asarray(v, np.float64)
    assert np.max(np.abs(np.asarray(v_new, np.float64) - bv)) <= 1e-3 * np.max(np.abs(upd))
    assert abs(loss - bl) <= 1e-5 * bl


def test_train_step_closed_form(oracle):
    # q = 0: P is uniform (1/S), out = column mean of V for every row; with
    # target 0 the loss is mean(out^2) and every row of grad_v is the same,
    # 2/(S*S*D) * sum_i out_i = 2/(S*D) * colmean(V).
    s, d, lr = 12, 5, 0.25
    v = synth.normal((s, d), seed=41, stream=1)
    out, v_new, loss = oracle.attention_train_step(np.zeros((s, d)), synth.normal((s, d), seed=41, stream=2), v,
                                                   np.zeros((s, d)), lr)
    cm = np.asarray(v, np.float64).mean(axis=0)
    np.testing.assert_allclose(out, np.tile(cm, (s, 1)), rtol=1e-5, atol=1e-6)
    assert abs(loss - float(np.mean(cm ** 2))) <= 1e-5 * float(np.mean(cm ** 2))
    np.testing.assert_allclose(v_new, np.asarray(v, np.float64) - lr * 2.0 / (s * d) * cm[None, :], rtol=1e-5,
                               atol=1e-6)


# --- sensitivity: planted mistakes are caught -----------------------------------

def test_checks_catch_planted_mistakes(oracle):
    s, d = 24, 16
    q, k, v = (synth.normal((s, d), seed=30, stream=i) for i in range(3))
    ref = _bf_attention(q, k, v, False)
    # transposed roles of Q and K, a missing scale, a wrong mask direction
    assert oracle_lib.normwise_rel(ref, oracle.attention(k, q, v)) > 1e-2
    assert oracle_lib.normwise_rel(ref, oracle.attention(q * np.sqrt(d), k, v)) > 1e-2
    assert oracle_lib.normwise_rel(_bf_attention(q, k, v, True), oracle.attention(q, k, v, False)) > 1e-2
    a, b = synth.uniform((8, 8), seed=31, stream=1), synth.uniform((8, 8), seed=31, stream=2)
    assert oracle_lib.normwise_rel(np.asarray(a, np.float64) @ b, oracle.matmul(a, b.T)) > 1e-2
    x, w = synth.normal((1, 2, 6, 6), seed=32, stream=1), synth.normal((3, 2, 3, 3), seed=32, stream=2)
    flipped = oracle.conv2d(x, w[:, :, ::-1, ::-1].copy(), None, (1, 1), (1, 1))
    assert oracle_lib.normwise_rel(_direct_conv(x, w, None, (1, 1), (1, 1), False), flipped) > 1e-2
    # train step: a sign error in the update and an untransposed P are caught
    t = synth.normal((s, d), seed=30, stream=5)
    _, bv, _ = _bf_train_step(q, k, v, t, 0.5, True)
    _, v_neg, _ = oracle.attention_train_step(q, k, v, t, -0.5, True)
    assert oracle_lib.normwise_rel(bv - v, np.asarray(v_neg, np.float64) - v) > 1e-2
    qq, kk = np.asarray(q, np.float64), np.asarray(k, np.float64)
    sc = np.where(np.triu(np.ones((s, s), bool), 1), -np.inf, qq @ kk.T / np.sqrt(d))
    pm = np.exp(sc - sc.max(axis=1, keepdims=True))
    pm /= pm.sum(axis=1, keepdims=True)
    go = 2.0 * (pm @ np.asarray(v, np.float64) - t) / (s * d)
    _, v_ok, _ = oracle.attention_train_step(q, k, v, t, 0.5, True)
    assert oracle_lib.normwise_rel(-0.5 * (pm @ go), np.asarray(v_ok, np.float64) - v) > 1e-2
