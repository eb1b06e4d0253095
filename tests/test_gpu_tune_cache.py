"""Tune caches on the hip device: first-call autotune, cache files, forced variants.

Mirrors the reference's tests/test_python_tune_cache_format_smoke.py:35-88:
v1-seeded cache files in the working directory are rewritten with the v2
header and a "#columns," line once a new shape is tuned.  Then every GEMM
variant and every attention split count is forced through a seeded cache on
odd shapes and checked against float64 / the oracle: the autotuner may pick
any of them.  Each case runs in a fresh interpreter (the caches are loaded
once per process) with its own working directory.
"""
import json
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

from gpu_util import note, require_hip
from lightning_core import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "lightining-core_amd")
TESTS = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def lc():
    return require_hip()


def _child(code, cwd, env=None):
    e = {k: v for k, v in os.environ.items() if not k.startswith("CJ_")}
    e.update(env or {})
    e["PYTHONPATH"] = os.pathsep.join([PKG, TESTS, e.get("PYTHONPATH", "")])
    note(f"[tune] child in {cwd} env={ {k: v for k, v in (env or {}).items()} }")
    r = subprocess.run([sys.executable, "-u", "-c", textwrap.dedent(code)], cwd=cwd, env=e, capture_output=True,
                       text=True, timeout=110)
    note("\n".join(l for l in r.stdout.splitlines() if not l.startswith("OUT"))[-3000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return r.stdout


def _lines(path):
    with open(path, encoding="utf-8") as f:
        return [l.rstrip("\n") for l in f if l.strip()]


def test_v1_seeded_caches_rewritten_after_autotune(lc, tmp_path):
    (tmp_path / ".lightning_core_matmul_tune_cache.csv").write_text("#lc_tune_cache,matmul,1\n64,64,64,16,1,0\n")
    (tmp_path / ".lightning_core_attn_tune_cache.csv").write_text("#lc_tune_cache,attention,1\nfwd,8,8,0,0,0,0\n")
    _child("""
        import numpy as np
        import lightning_core as lc
        rng = np.random.default_rng(7)
        a = (rng.standard_normal((16, 16)) * 0.2).astype(np.float32)
        b = (rng.standard_normal((16, 16)) * 0.2).astype(np.float32)
        c = lc.matmul2d(a, b, device="hip")
        assert np.abs(c - a.astype(np.float64) @ b).max() < 1e-5
        q, k, v = ((rng.standard_normal((16, 16)) * 0.2).astype(np.float32) for _ in range(3))
        o = np.asarray(lc.attention2d(q, k, v, causal=False, device="hip")).reshape(16, 16)
        s = q.astype(np.float64) @ k.T / 4.0
        p = np.exp(s - s.max(1, keepdims=True)); p /= p.sum(1, keepdims=True)
        assert np.abs(o - p @ v).max() < 1e-5
        # a 256 x 64 train step fills a T row (autotuned dV splits)
        sess = lc.AttentionSession(256, 64, causal=True)
        q, k, v, t = ((rng.standard_normal((256, 64))).astype(np.float32) for _ in range(4))
        sess.train_step(q, k, v, t, 0.5)
        sess.close()
        print("ok")
    """, tmp_path)
    mm = _lines(tmp_path / ".lightning_core_matmul_tune_cache.csv")
    at = _lines(tmp_path / ".lightning_core_attn_tune_cache.csv")
    note(f"[tune] matmul cache: {mm}")
    note(f"[tune] attention cache: {at}")
    assert mm[0] == "#lc_tune_cache,matmul,2" and mm[1].startswith("#columns,")
    assert at[0] == "#lc_tune_cache,attention,2" and at[1].startswith("#columns,")
    assert "64,64,64,16,1,0" in mm  # the reference-layout row is kept
    assert any(r.startswith("16,16,16,0,gfx950,f32_") for r in mm)
    assert any(r.startswith("HF,16,16,0,") and ",gfx950," in r for r in at)
    assert any(r.startswith("HT,256,64,1,") and ",gfx950," in r for r in at)


F32_CASES = [("f32_dp_64x64x64", (100, 130, 77)), ("f32_streamk_64x64x64", (257, 300, 64)),
             ("f32_dp_64x64x32", (1000, 777, 1030)), ("f32_streamk_64x64x64", (1000, 777, 1030))]
HALF_CASES = [("half_w4_256x256", (300, 129, 200)), ("half_w4_256x256", (520, 256, 130)),
              ("half_w4d_256x256", (300, 129, 200)), ("half_w4d_256x256", (520, 64, 130)),
              ("half_w4r_256x256", (300, 129, 200)), ("half_w4r_256x256", (520, 64, 130)),
              ("half_w4r_256x256", (700, 1000, 513)),
              ("half_w4h_256x256", (300, 129, 200)), ("half_w4h_256x256", (520, 64, 130)),
              ("half_w4h_256x256", (700, 1000, 513)), ("half_w4h_256x256", (256, 1728, 512)),
              ("half_lds_256x256", (300, 129, 200)), ("half_big8_256x256", (300, 129, 200)),
              ("half_big4_256x256", (520, 256, 130)), ("half_mid_128x128", (77, 320, 513)),
              ("half_small_64x64", (1000, 777, 1030)), ("half_skinny_16x64", (9, 200, 300))]
_TILES = {"f32_dp_64x64x64": "64,64,64,8,2", "f32_streamk_64x64x64": "64,64,64,8,2",
          "f32_dp_64x64x32": "64,64,32,8,2", "half_w4_256x256": "256,256,32,4,1",
          "half_w4d_256x256": "256,256,64,4,1", "half_w4r_256x256": "256,256,64,4,1",
          "half_w4h_256x256": "256,256,64,4,1",
          "half_lds_256x256": "256,256,64,8,1",
          "half_big8_256x256": "256,256,64,8,1", "half_big4_256x256": "256,256,64,4,1",
          "half_mid_128x128": "128,128,64,4,1", "half_small_64x64": "64,64,64,4,1",
          "half_skinny_16x64": "16,64,256,8,2"}


@pytest.mark.parametrize("dtype,cases", [("f32", F32_CASES), ("bf16", HALF_CASES), ("f16", HALF_CASES)])
def test_forced_gemm_variants(lc, tmp_path, dtype, cases):
    # one seeded cache per (variant, shape), loaded in turn by one child
    code = {"f32": 0, "bf16": 1, "f16": 2}[dtype]
    jobs = []
    for name, (m, k, n) in cases:
        cache = tmp_path / f"mm_{name}_{m}_{k}_{n}.csv"
        cache.write_text("#lc_tune_cache,matmul,2\n" + f"{m},{k},{n},{code},gfx950,{name},{_TILES[name]}\n")
        jobs.append((str(cache), name, m, k, n))
    before = {j[0]: open(j[0]).read() for j in jobs}
    out = _child(f"""
        import numpy as np
        import lightning_core as lc
        from lightning_core import synth
        for cache, name, m, k, n in {jobs!r}:
            print("[case]", name, m, k, n, flush=True)
            lc.tune_cache_load(cache)
            a = synth.normal((m, k), stream=11)
            b = synth.normal((k, n), stream=12)
            sess = lc.MatMulResidentSession(m, k, n, compute_dtype={dtype!r})
            c = np.zeros(m * n, np.float32)
            sess.start_into(a, b, c)
            sess.finish_into(out=c)
            sess.close()
            ar, br = synth.round_to(a, {dtype!r}), synth.round_to(b, {dtype!r})
            ref = ar.astype(np.float64) @ br.astype(np.float64)
            err = np.abs(c.reshape(m, n) - ref).max() / np.abs(ref).max()
            print("ERR", name, err, flush=True)
    """, tmp_path)
    tol = 1e-4 if dtype == "f32" else 2e-2
    errs = [l.split() for l in out.splitlines() if l.startswith("ERR")]
    assert len(errs) == len(jobs)
    for _, name, err in errs:
        note(f"[parity] forced {name} {dtype} normwise={float(err):.3e}")
        assert float(err) <= tol, name
    for path, text in before.items():
        assert open(path).read() == text  # the cached entry was used, not re-tuned


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_w4_gemm_matches_lds_bitwise(lc, tmp_path, dtype):
    # The 4-wave kernels (ring of 32-deep slices; two 64-deep stages; ring
    # of 128-byte-row parts, with the barrier at the end or in the middle of
    # a stage) accumulate every output in the same k order as the 8-wave
    # kernel: forced one after the other on the same inputs, the five must
    # agree bit for bit (ragged M / N / K, one and many k stages, more stages
    # than ring slots, stage counts that are and are not multiples of w4h's
    # five-stage unroll).
    code = {"bf16": 1, "f16": 2}[dtype]
    shapes = [(600, 320, 700), (1100, 1024, 1300), (257, 64, 255), (300, 1728, 260)]
    jobs = []
    for m, k, n in shapes:
        for name in ("half_lds_256x256", "half_w4_256x256", "half_w4d_256x256", "half_w4r_256x256",
                     "half_w4h_256x256"):
            cache = tmp_path / f"mm_{name}_{m}_{k}_{n}.csv"
            cache.write_text("#lc_tune_cache,matmul,2\n" + f"{m},{k},{n},{code},gfx950,{name},{_TILES[name]}\n")
            jobs.append((str(cache), name, m, k, n))
    out = _child(f"""
        import hashlib
        import numpy as np
        import lightning_core as lc
        from lightning_core import synth
        for cache, name, m, k, n in {jobs!r}:
            print("[case]", name, m, k, n, flush=True)
            lc.tune_cache_load(cache)
            a = synth.normal((m, k), stream=31)
            b = synth.normal((k, n), stream=32)
            sess = lc.MatMulResidentSession(m, k, n, compute_dtype={dtype!r})
            c = np.zeros(m * n, np.float32)
            sess.start_into(a, b, c)
            sess.finish_into(out=c)
            sess.close()
            print("SHA", name, m, k, n, hashlib.sha256(c.tobytes()).hexdigest(), float(np.abs(c).max()), flush=True)
    """, tmp_path)
    sums = {}
    for line in out.splitlines():
        if line.startswith("SHA"):
            _, name, m, k, n, digest, amax = line.split()
            assert float(amax) > 0.0
            sums.setdefault((m, k, n), {})[name] = digest
    assert len(sums) == len(shapes)
    for shape, by_name in sums.items():
        note(f"[parity] w4 / w4d / w4r / w4h vs lds {dtype} {shape}: "
             f"{'identical' if len(set(by_name.values())) == 1 else 'DIFFER'}")
        assert by_name["half_w4_256x256"] == by_name["half_lds_256x256"], shape
        assert by_name["half_w4r_256x256"] == by_name["half_lds_256x256"], shape
        assert by_name["half_w4d_256x256"] == by_name["half_lds_256x256"], shape
        assert by_name["half_w4h_256x256"] == by_name["half_lds_256x256"], shape


@pytest.mark.parametrize("s,d,causal", [(256, 64, False), (200, 48, True), (130, 96, False), (256, 64, True),
                                        (1000, 64, False), (33, 20, True), (17, 8, False)])
def test_forced_attention_splits(lc, oracle, tmp_path, s, d, causal):
    # 16 selects the 16-query kernel where D <= 64 and D % 4 == 0 (and the
    # heuristic split elsewhere, e.g. D = 96); S = 1000 gives its waves four
    # key tiles each (the register prefetch path), S = 17 / 33 ragged blocks.
    caches = []
    for ks in (1, 2, 4, 8, 16):
        cache = tmp_path / f"attn_{ks}.csv"
        cache.write_text("#lc_tune_cache,attention,2\n" + f"HF,{s},{d},{int(causal)},0,0,gfx950,{ks}\n"
                         + f"HF,{s},{d},{int(causal)},0,1,gfx950,{ks}\n")
        caches.append((ks, str(cache)))
    out = _child(f"""
        import json
        import numpy as np
        import lightning_core as lc
        from lightning_core import synth
        q, k, v = (synth.normal(({s}, {d}), stream=60 + i) for i in range(3))
        for ks, cache in {caches!r}:
            print("[case] splits", ks, flush=True)
            lc.attention_tune_cache_load(cache)
            o = np.asarray(lc.attention2d(q, k, v, causal={causal}, device="hip"))
            print("OUT", ks, json.dumps(o.ravel().tolist()), flush=True)
    """, tmp_path)
    q, k, v = (synth.normal((s, d), stream=60 + i) for i in range(3))
    ref = np.asarray(oracle.attention(q, k, v, causal)).ravel()
    outs = [l for l in out.splitlines() if l.startswith("OUT")]
    assert len(outs) == 5
    for line in outs:
        _, ks, payload = line.split(" ", 2)
        got = np.asarray(json.loads(payload), np.float32)
        err = np.abs(got - ref).max() / np.abs(ref).max()
        note(f"[parity] forced attention splits={ks} S={s} D={d} causal={causal} normwise={err:.3e}")
        assert err <= 1e-4


@pytest.mark.parametrize("s,d,causal", [(256, 64, False), (100, 32, True), (1000, 64, False), (33, 20, True)])
def test_forced_train_dv_splits(lc, oracle, tmp_path, s, d, causal):
    """Every dV variant of the train step, forced through HT rows (16: the
    16-key-block kernel), against the oracle's step: updated V, output, loss."""
    caches = []
    for ks in (1, 2, 4, 8, 16):
        cache = tmp_path / f"train_{ks}.csv"
        rows = [f"HT,{s},{d},{int(causal)},{rh},{sy},{cl},gfx950,{ks}"
                for rh in (0, 1) for sy in (0, 1) for cl in (0, 1)]
        cache.write_text("#lc_tune_cache,attention,2\n" + "\n".join(rows) + "\n")
        caches.append((ks, str(cache)))
    lr = 3.0
    out = _child(f"""
        import json
        import numpy as np
        import lightning_core as lc
        from lightning_core import synth
        q, k, v, t = (synth.normal(({s}, {d}), stream=700 + i) for i in range(4))
        for ks, cache in {caches!r}:
            print("[case] dV splits", ks, flush=True)
            lc.attention_tune_cache_load(cache)
            sess = lc.AttentionSession({s}, {d}, causal={causal})
            o, vn, loss = sess.train_step(q, k, v.copy(), t, {lr})
            sess.close()
            print("OUT", ks, json.dumps([np.asarray(vn).ravel().tolist(), np.asarray(o).ravel().tolist(),
                                         float(loss)]), flush=True)
    """, tmp_path)
    q, k, v, t = (synth.normal((s, d), stream=700 + i) for i in range(4))
    ref_out, ref_v, ref_loss = oracle.attention_train_step(q, k, v, t, lr, causal)
    outs = [l for l in out.splitlines() if l.startswith("OUT")]
    assert len(outs) == 5
    for line in outs:
        _, ks, payload = line.split(" ", 2)
        vn, o, loss = json.loads(payload)
        vn = np.asarray(vn, np.float64)
        o = np.asarray(o, np.float32)
        # the V check is relative to the update (V itself is much larger), as
        # in test_gpu_attention_train.py
        v0 = np.asarray(v, np.float64).ravel()
        vr = np.asarray(ref_v, np.float64).ravel()
        upd = np.abs(vr - v0).max()
        ev = np.abs(vn - vr).max()
        eo = np.abs(o - np.asarray(ref_out).ravel()).max() / np.abs(np.asarray(ref_out)).max()
        note(f"[parity] forced dV splits={ks} S={s} D={d} causal={causal} v err {ev / upd:.2e} of the update, "
             f"out={eo:.3e}, loss {loss:.6g} vs {float(ref_loss):.6g}")
        assert ev <= 1e-3 * upd + 4 * np.finfo(np.float32).eps * np.abs(v0).max()
        assert eo <= 1e-4
        assert abs(loss - float(ref_loss)) <= 1e-4 * abs(float(ref_loss))
