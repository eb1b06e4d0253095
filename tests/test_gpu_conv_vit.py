"""conv2d, the conv -> attention pipeline and the ViT block on the hip device.

conv2d vs the oracle's im2col path (core/ops.hpp:855-1213) on the golden
vectors and extra geometries; conv_attention_torchstrong_nchw vs the golden
vectors of bind_integrated.cpp:614-730 (flat slices and QkvPackRepeat);
the ViT block (fp16) vs the oracle composition on the
rows of two whole images (every stage of those images is exercised).
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


@pytest.mark.parametrize("case", oracle_lib.golden_cases("conv_"), ids=lambda c: c["name"])
def test_conv_golden(lc, case):
    p = case["params"]
    x = oracle_lib.golden_input(case, "x").reshape(p["batch"], p["in_c"], p["in_h"], p["in_w"])
    w = oracle_lib.golden_input(case, "w").reshape(p["out_c"], p["in_c"], p["kh"], p["kw"])
    bias = oracle_lib.golden_input(case, "bias")
    exp = np.asarray(case["expected"], np.float32)
    if p["op"] == "conv2d_nchw":
        got = lc.conv2d_nchw(x, w, bias, p["stride_h"], p["stride_w"], p["pad_h"], p["pad_w"],
                             apply_relu=p["relu"]).ravel()
        assert oracle_lib.elementwise_ok(exp, got, 1.5e-2, 1.5e-2)
    else:
        got = lc.api.conv_attention_torchstrong_nchw(x, w, bias, p["seq_len"], p["head_dim"], p["stride_h"],
                                                     p["stride_w"], p["pad_h"], p["pad_w"])
    assert_parity(exp, got, "f32", case["name"])


@pytest.mark.parametrize("xs,ws,stride,pad", [((2, 3, 17, 19), (5, 3, 3, 3), (1, 1), (1, 1)),
                                              ((1, 4, 16, 16), (8, 4, 1, 1), (1, 1), (0, 0)),
                                              ((2, 3, 64, 64), (16, 3, 16, 16), (16, 16), (0, 0))])
def test_conv_extra(lc, oracle, xs, ws, stride, pad):
    x, w = synth.normal(xs, stream=1), synth.normal(ws, stream=2)
    bias = synth.normal((ws[0],), stream=3)
    for relu in (False, True):
        got = lc.conv2d_nchw(x, w, bias, stride[0], stride[1], pad[0], pad[1], apply_relu=relu)
        assert_parity(oracle.conv2d(x, w, bias, stride, pad, relu), got, "f32", f"conv {xs} {ws} relu={relu}")


# The reference's own conv -> attention hotspot shapes (README.md Pipeline
# Bench: conv n=1 c=3->16 h=w=8 k=3 (pad 1) + attention seq 48/96/192, d
# 48/8), served by the fused one-launch kernel, plus shapes whose conv output
# exceeds the fused kernel's 8192 values (the im2col + GEMM + repeat chain).
# Fused variants: a strided / unpadded non-3x3 kernel, 3x3 with stride 2 and
# batch 2 (pixel count not a multiple of 64), 4 input channels unpadded, an
# input too large to stage in LDS (read from global memory), and 5 input
# channels (the general conv loop).
@pytest.mark.parametrize("xs,ws,stride,pad,seq,hd", [
    ((1, 3, 8, 8), (16, 3, 3, 3), (1, 1), (1, 1), 48, 48),
    ((1, 3, 8, 8), (16, 3, 3, 3), (1, 1), (1, 1), 192, 48),
    ((1, 3, 8, 8), (16, 3, 3, 3), (1, 1), (1, 1), 192, 8),
    ((1, 3, 8, 8), (16, 3, 3, 3), (1, 1), (1, 1), 96, 48),
    ((2, 3, 33, 31), (16, 3, 3, 3), (1, 1), (1, 1), 100, 64),
    ((1, 4, 40, 40), (24, 4, 3, 3), (1, 1), (1, 1), 64, 200),
    ((1, 2, 9, 11), (5, 2, 3, 2), (2, 1), (0, 0), 30, 7),
    ((2, 1, 15, 13), (6, 1, 3, 3), (2, 2), (1, 1), 40, 24),
    ((1, 4, 12, 10), (7, 4, 3, 3), (1, 1), (0, 0), 33, 20),
    ((1, 4, 64, 64), (8, 4, 3, 3), (4, 4), (1, 1), 64, 32),
    ((1, 5, 8, 8), (16, 5, 3, 3), (1, 1), (1, 1), 48, 48),
    ((1, 3, 8, 8), (16, 3, 3, 3), (1, 1), (1, 1), 40, 100),
])
def test_conv_attention_shapes(lc, oracle, xs, ws, stride, pad, seq, hd):
    x, w = synth.normal(xs, stream=40), synth.normal(ws, std=0.3, stream=41)
    bias = synth.normal((ws[0],), stream=42)
    got = lc.api.conv_attention_torchstrong_nchw(x, w, bias, seq, hd, stride[0], stride[1], pad[0], pad[1])
    ref = oracle.conv_attention(x, w, bias, seq, hd, stride, pad)
    assert_parity(ref.ravel(), got, "f32", f"conv_attention {xs} {ws} seq={seq} d={hd}")


# The fused calls return when their kernel's last workgroup raises a
# host-mapped completion flag (no stream sync).  Back-to-back calls with
# fresh inputs, cycling through shapes of both fused kernels (16-query D <= 64,
# 32-query D > 64) and both execution modes, must each return the result of
# their own inputs: an output read before the kernel's stores were visible
# would show the previous call's values.
def test_conv_attention_repeated_calls_see_their_own_results(lc, oracle):
    shapes = [(48, 48), (192, 8), (40, 100), (96, 48)]
    for it in range(48):
        seq, hd = shapes[it % len(shapes)]
        mode = "eager" if (it // len(shapes)) % 2 == 0 else "graph"
        x = synth.normal((1, 3, 8, 8), stream=700 + it)
        w = synth.normal((16, 3, 3, 3), std=0.3, stream=800 + it)
        bias = synth.normal((16,), stream=900 + it)
        got = lc.api.conv_attention_torchstrong_nchw(x, w, bias, seq, hd, 1, 1, 1, 1, execution_mode=mode)
        ref = oracle.conv_attention(x, w, bias, seq, hd, (1, 1), (1, 1))
        assert_parity(ref.ravel(), got, "f32", f"call {it} {mode} seq={seq} d={hd}")


# Graph mode: one HIP graph per shape key, replayed.  Each case replays it four
# times with fresh inputs, an eager call (and its stream sync) between the
# replays, and checks every replay bit for bit against the eager result (same
# kernels, same arithmetic), plus the oracle once.  Shapes: the fused kernel
# reading mapped staging, the fused kernel with an input too large to stage
# (device copies in the graph), and the unfused im2col / GEMM / repeat chain.
@pytest.mark.parametrize("xs,ws,stride,pad,seq,hd,with_bias", [
    ((1, 3, 8, 8), (16, 3, 3, 3), (1, 1), (1, 1), 48, 48, True),
    ((1, 3, 8, 8), (16, 3, 3, 3), (1, 1), (1, 1), 192, 8, False),
    ((1, 4, 64, 64), (8, 4, 3, 3), (4, 4), (1, 1), 64, 32, True),
    ((2, 3, 33, 31), (16, 3, 3, 3), (1, 1), (1, 1), 100, 64, True),
    ((1, 3, 40, 40), (24, 3, 3, 3), (1, 1), (1, 1), 64, 200, False),
])
def test_conv_attention_graph_replays(lc, oracle, xs, ws, stride, pad, seq, hd, with_bias):
    for it in range(4):
        x, w = synth.normal(xs, stream=600 + it), synth.normal(ws, std=0.3, stream=610 + it)
        bias = synth.normal((ws[0],), stream=620 + it) if with_bias else None
        note(f"[graph] {xs} {ws} seq={seq} d={hd} bias={with_bias} replay {it}")
        g = lc.api.conv_attention_torchstrong_nchw(x, w, bias, seq, hd, stride[0], stride[1], pad[0], pad[1],
                                                   execution_mode="graph")
        e = lc.api.conv_attention_torchstrong_nchw(x, w, bias, seq, hd, stride[0], stride[1], pad[0], pad[1],
                                                   execution_mode="eager")
        np.testing.assert_array_equal(g, e)
        if it == 0:
            ref = oracle.conv_attention(x, w, bias, seq, hd, stride, pad)
            assert_parity(ref.ravel(), g, "f32", f"graph conv_attention {xs} {ws} seq={seq} d={hd}")


def test_conv_attention_graph_non3x3_fallback_and_strict(lc, monkeypatch):
    x, w = synth.normal((1, 2, 9, 11), stream=630), synth.normal((5, 2, 3, 2), std=0.3, stream=631)
    e = lc.api.conv_attention_torchstrong_nchw(x, w, None, 30, 7, 2, 1, 0, 0, execution_mode="eager")
    monkeypatch.delenv("LC_GRAPH_MODE_STRICT", raising=False)
    g = lc.api.conv_attention_torchstrong_nchw(x, w, None, 30, 7, 2, 1, 0, 0, execution_mode="graph")
    np.testing.assert_array_equal(g, e)  # the reference's fallback contract: the eager result
    monkeypatch.setenv("LC_GRAPH_MODE_STRICT", "1")
    with pytest.raises(RuntimeError, match="3x3 conv weights"):
        lc.api.conv_attention_torchstrong_nchw(x, w, None, 30, 7, 2, 1, 0, 0, execution_mode="graph")


def test_conv_attention_ab_report_and_cache(lc):
    lc.api.clear_conv_attention_graph_cache()
    assert lc._core._lib().lcConvAttentionGraphCacheSize() == 0
    x, w = synth.normal((1, 3, 8, 8), stream=640), synth.normal((16, 3, 3, 3), std=0.3, stream=641)
    b = synth.normal((16,), stream=642)
    rep = lc.api.conv_attention_torchstrong_nchw_ab_report(x, w, b, 96, 48, 1, 1, 1, 1, warmup=2, repeat=10)
    note(f"[graph] ab report {rep}")
    assert rep["allclose"] and rep["max_abs_diff"] == 0.0
    assert rep["winner"] in ("graph", "eager", "tie") and rep["eager_ms"] > 0 and rep["graph_ms"] > 0
    assert lc._core._lib().lcConvAttentionGraphCacheSize() == 1
    lc.api.clear_conv_attention_graph_cache()
    assert lc._core._lib().lcConvAttentionGraphCacheSize() == 0


def test_conv_attention_graph_mode_matches_eager(lc):
    x, w = synth.normal((1, 3, 8, 8), stream=4), synth.normal((8, 3, 3, 3), stream=5)
    e = lc.api.conv_attention_torchstrong_nchw(x, w, None, 16, 16, 1, 1, 1, 1, execution_mode="eager")
    g = lc.api.conv_attention_torchstrong_nchw(x, w, None, 16, 16, 1, 1, 1, 1, execution_mode="graph")
    np.testing.assert_array_equal(e, g)


def _vit_inputs(bn, c, img, p, e):
    x = synth.uniform((bn, c, img, img), lo=0.0, hi=1.0, stream=30)
    w_conv = synth.normal((e, c, p, p), std=0.02, stream=31)
    w_qkv = synth.normal((e, 3 * e), std=0.02, stream=32)
    w_o = synth.normal((e, e), std=0.02, stream=33)
    return x, w_conv, w_qkv, w_o


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_vit_block_small(lc, oracle, dtype):
    bn, c, img, p, e, heads = 2, 3, 64, 16, 128, 2
    x, w_conv, w_qkv, w_o = _vit_inputs(bn, c, img, p, e)
    got = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype=dtype)
    ref = oracle.vit_block(*(synth.round_to(t, dtype) for t in (x, w_conv, w_qkv, w_o)), heads)
    assert_parity(ref, got.reshape(ref.shape), dtype, f"vit small {dtype}")


# Shapes for the ring-pipelined ViT GEMMs: P = 8 and 32 patch sources, token
# counts that are not tile multiples (rows clamped), and T % 4 != 0, which
# sends the QKV projection to the element-wise epilogue.
@pytest.mark.parametrize("bn,img,p,e,heads,dtype", [
    (3, 40, 8, 128, 2, "f16"),     # T = 25 (T % 4 != 0), M = 75
    (5, 96, 16, 192, 3, "bf16"),   # T = 36, M = 180, three heads of 64
    (2, 64, 32, 128, 1, "f16"),    # P = 32, T = 4, one head of 128
    (1, 48, 16, 128, 2, "bf16"),   # M = 9, a single partial tile
])
def test_vit_block_shapes(lc, oracle, bn, img, p, e, heads, dtype):
    note(f"[case] vit bn={bn} img={img} p={p} e={e} heads={heads} {dtype}")
    x, w_conv, w_qkv, w_o = _vit_inputs(bn, 3, img, p, e)
    got = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype=dtype)
    ref = oracle.vit_block(*(synth.round_to(t, dtype) for t in (x, w_conv, w_qkv, w_o)), heads)
    assert_parity(ref, got.reshape(ref.shape), dtype, f"vit {bn}x{img} p{p} e{e} {dtype}")


def test_vit_block_ring_off_matches(lc, monkeypatch):
    # CJ_HIP_VIT_RING=0 keeps the register-staged GEMMs: same inputs, results
    # within the 16-bit tolerance of the ring path (the k order of the
    # accumulation is the same; only the tiling differs).
    bn, c, img, p, e, heads = 2, 3, 64, 16, 128, 2
    x, w_conv, w_qkv, w_o = _vit_inputs(bn, c, img, p, e)
    ring = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype="f16")
    monkeypatch.setenv("CJ_HIP_VIT_RING", "0")
    plain = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype="f16")
    assert np.abs(ring - plain).max() <= 2e-2 * np.abs(plain).max()


@pytest.mark.parametrize("p,e", [(16, 128), (32, 256), (8, 128)])
def test_vit_block_ring_stage_depth_bitwise(lc, monkeypatch, p, e):
    # The patch and output GEMMs take 128-deep ring stages when K allows
    # (CJ_HIP_VIT_RING_BK=64 forces 64): same k order, so the same bits.  P = 8
    # keeps 64-deep stages for the patch GEMM (a 128-deep stage would span
    # two channels) and checks that path too.
    bn, c, img, heads = 2, 3, 64, 2
    x, w_conv, w_qkv, w_o = _vit_inputs(bn, c, img, p, e)
    deep = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype="f16")
    monkeypatch.setenv("CJ_HIP_VIT_RING_BK", "64")
    shallow = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype="f16")
    np.testing.assert_array_equal(deep, shallow)


# The fused QKV-projection + attention kernel (default where head dim is 64
# and T <= 224) against the separate QKV GEMM and attention kernels
# (CJ_HIP_VIT_FUSED=0): the projection accumulates in the same k order and the
# attention runs the same per-wave arithmetic, so the bits match.  T = 25, 9
# and 169 are not multiples of 4 or 64; T = 196 is config 4's.
@pytest.mark.parametrize("bn,img,p,e,heads,dtype", [
    (2, 64, 16, 128, 2, "f16"),    # T = 16
    (3, 40, 8, 128, 2, "f16"),     # T = 25
    (5, 96, 16, 192, 3, "bf16"),   # T = 36
    (1, 48, 16, 128, 2, "bf16"),   # T = 9
    (1, 208, 16, 128, 2, "f16"),   # T = 169
    (2, 224, 16, 768, 12, "bf16"),  # config 4's image and width, T = 196
])
def test_vit_block_fused_matches_unfused(lc, monkeypatch, bn, img, p, e, heads, dtype):
    note(f"[case] vit fused vs unfused bn={bn} img={img} p={p} e={e} heads={heads} {dtype}")
    x, w_conv, w_qkv, w_o = _vit_inputs(bn, 3, img, p, e)
    fused = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype=dtype)
    monkeypatch.setenv("CJ_HIP_VIT_FUSED", "0")
    unfused = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype=dtype)
    np.testing.assert_array_equal(fused, unfused)


# The fused kernel's edges: one 64-deep k-stage (E = 64, one head) and the
# largest token count it takes (T = 224 = 14 x 16 patches of a 224 x 256
# image: seven full query blocks, keys 224..255 padding), each bit-identical to
# the separate kernels and, for T = 224, against the oracle on the whole block.
@pytest.mark.parametrize("bn,ih,iw,p,e,heads,dtype", [
    (2, 32, 32, 8, 64, 1, "f16"),     # T = 16, E = 64
    (1, 224, 256, 16, 128, 2, "bf16"),  # T = 224
])
def test_vit_block_fused_edges(lc, oracle, monkeypatch, bn, ih, iw, p, e, heads, dtype):
    note(f"[case] vit fused edges bn={bn} {ih}x{iw} p={p} e={e} heads={heads} {dtype}")
    x = synth.uniform((bn, 3, ih, iw), lo=0.0, hi=1.0, stream=34)
    w_conv = synth.normal((e, 3, p, p), std=0.02, stream=35)
    w_qkv = synth.normal((e, 3 * e), std=0.02, stream=36)
    w_o = synth.normal((e, e), std=0.02, stream=37)
    fused = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype=dtype)
    ref = oracle.vit_block(*(synth.round_to(t, dtype) for t in (x, w_conv, w_qkv, w_o)), heads)
    assert_parity(ref, fused.reshape(ref.shape), dtype, f"vit fused {ih}x{iw} e{e} {dtype}")
    monkeypatch.setenv("CJ_HIP_VIT_FUSED", "0")
    unfused = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype=dtype)
    np.testing.assert_array_equal(fused, unfused)


# The input stored as patch rows with the patch conv as a row-major GEMM (the
# default) against the implicit-im2col GEMM on the NCHW image
# (CJ_HIP_VIT_PATCHIFY=0): same tiles and k order, so the same bits.  Shapes:
# P = 8, 16 and 32, an image that is not a multiple of the patch (the last
# 8 columns and rows are not covered), non-square.
@pytest.mark.parametrize("bn,ih,iw,p,e,heads,dtype", [
    (2, 64, 64, 16, 128, 2, "f16"),
    (3, 40, 48, 8, 128, 2, "bf16"),
    (2, 64, 64, 32, 256, 2, "f16"),
    (1, 56, 40, 16, 128, 1, "bf16"),
])
def test_vit_block_patch_rows_bitwise(lc, monkeypatch, bn, ih, iw, p, e, heads, dtype):
    note(f"[case] vit patch rows bn={bn} {ih}x{iw} p={p} e={e} heads={heads} {dtype}")
    x = synth.uniform((bn, 3, ih, iw), lo=0.0, hi=1.0, stream=38)
    w_conv = synth.normal((e, 3, p, p), std=0.02, stream=39)
    w_qkv = synth.normal((e, 3 * e), std=0.02, stream=40)
    w_o = synth.normal((e, e), std=0.02, stream=41)
    rows = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype=dtype)
    monkeypatch.setenv("CJ_HIP_VIT_PATCHIFY", "0")
    nchw = lc.vit_block(x, w_conv, w_qkv, w_o, heads, compute_dtype=dtype)
    np.testing.assert_array_equal(rows, nchw)


def test_vit_block_config4(lc, oracle):
    bn, c, img, p, e, heads = 8, 3, 224, 16, 768, 12
    note("[case] config 4 ViT block")
    x, w_conv, w_qkv, w_o = _vit_inputs(bn, c, img, p, e)
    s = lc.VitBlockSession(bn, c, img, img, p, e, heads, "f16")
    s.set_weights(w_conv, w_qkv, w_o)
    got = s.forward(x)
    s.run_cached(3)
    again = s.forward(None)
    np.testing.assert_array_equal(got, again)  # deterministic, resident input
    t = s.tokens
    xr, wcr, wqr, wor = (synth.round_f16(a) for a in (x, w_conv, w_qkv, w_o))
    for img_idx in (0, bn - 1):
        rows = (img_idx * t, (img_idx + 1) * t)
        ref = oracle.vit_block(xr, wcr, wqr, wor, heads, rows=rows)
        assert_parity(ref, got.reshape(bn * t, e)[rows[0]:rows[1]], "f16", f"config4 image {img_idx}")
