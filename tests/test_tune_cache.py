"""Tune-cache file formats and the CJ_* runtime profile autoload (no GPU).

The caches follow the reference's convention (src/ops/matmul_metal.mm:133-139,
:416-517; src/attention_metal.mm:184-336): "#lc_tune_cache,<kind>,<version>",
a "#columns," line, CSV rows; versions 1-2 read, 2 written, a foreign header
clears the table.  The reference's own smoke test seeds v1 files
(tests/test_python_tune_cache_format_smoke.py:40-60); the same seeds are used
here.  The runtime profile follows src/runtime.cpp:101-168.

Both are process-global state, so each case runs in a fresh interpreter.
"""
import os
import subprocess
import sys
import textwrap

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "lightining-core_amd")


def _run(code, cwd, env=None):
    e = dict(os.environ)
    for k in list(e):
        if k.startswith("CJ_"):
            del e[k]
    e.update(env or {})
    e["PYTHONPATH"] = PKG + os.pathsep + e.get("PYTHONPATH", "")
    r = subprocess.run([sys.executable, "-c", textwrap.dedent(code)], cwd=cwd, env=e, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def _lines(path):
    with open(path, encoding="utf-8") as f:
        return [l.rstrip("\n") for l in f if l.strip()]


def test_matmul_cache_v1_seed_is_read_and_rewritten_as_v2(tmp_path):
    seed = tmp_path / "seed.csv"
    seed.write_text("#lc_tune_cache,matmul,1\n64,64,64,16,1,0\n", encoding="utf-8")
    out = tmp_path / "out.csv"
    _run(f"""
        import lightning_core as lc
        lc.tune_cache_load({str(seed)!r})
        assert lc.tune_cache_size() == 0  # a Metal row: kept, not a gfx950 entry
        lc.tune_cache_save({str(out)!r})
    """, tmp_path)
    lines = _lines(out)
    assert lines[0] == "#lc_tune_cache,matmul,2"
    assert lines[1].startswith("#columns,m,k,n,dtype,arch,kernel")
    assert "64,64,64,16,1,0" in lines[2:]  # the reference's row survives the rewrite


def test_matmul_cache_v2_round_trip_and_bad_rows(tmp_path):
    src = tmp_path / "in.csv"
    src.write_text("\n".join([
        "#lc_tune_cache,matmul,2",
        "#columns,m,k,n,dtype,arch,kernel,tile_m,tile_n,tile_k,waves,split_k",
        "1024,1024,1024,0,gfx950,f32_dp_64x64x64,64,64,64,8,2",
        "4096,4096,4096,1,gfx950,half_lds_256x256,256,256,64,8,1",
        "12,13,14,2,gfx950,half_skinny_16x64,16,64,256,8,2",
        "1,2,3,0,gfx950,broken,x,64,64,8,2",   # malformed: ignored
        "1,2,3",                                # short: ignored
    ]) + "\n", encoding="utf-8")
    out = tmp_path / "out.csv"
    _run(f"""
        import lightning_core as lc
        lc.tune_cache_load({str(src)!r})
        assert lc.tune_cache_size() == 3, lc.tune_cache_size()
        lc.tune_cache_save({str(out)!r})
        lc.matmul_reset_tuning()
        assert lc.tune_cache_size() == 0
    """, tmp_path)
    rows = _lines(out)[2:]
    assert sorted(rows) == sorted([
        "1024,1024,1024,0,gfx950,f32_dp_64x64x64,64,64,64,8,2",
        "4096,4096,4096,1,gfx950,half_lds_256x256,256,256,64,8,1",
        "12,13,14,2,gfx950,half_skinny_16x64,16,64,256,8,2",
    ])


def test_cache_foreign_header_clears(tmp_path):
    bad = tmp_path / "bad.csv"
    bad.write_text("#lc_tune_cache,matmul,3\n1024,1024,1024,0,gfx950,f32_dp_64x64x64,64,64,64,8,2\n",
                   encoding="utf-8")
    other = tmp_path / "other.csv"
    other.write_text("#lc_tune_cache,attention,2\nF,256,64,0,0,0,2\n", encoding="utf-8")
    good = tmp_path / "good.csv"
    good.write_text("#lc_tune_cache,matmul,2\n8,8,8,0,gfx950,f32_streamk_64x64x64,64,64,64,8,2\n",
                    encoding="utf-8")
    _run(f"""
        import lightning_core as lc
        lc.tune_cache_load({str(good)!r})
        assert lc.tune_cache_size() == 1
        for path in ({str(bad)!r}, {str(other)!r}):
            try:
                lc.tune_cache_load(path)
            except lc.LightningCoreError as e:
                assert "header" in str(e)
            else:
                raise AssertionError("a foreign header must be rejected")
            assert lc.tune_cache_size() == 0  # and the table cleared
        try:
            lc.tune_cache_load({str(tmp_path / "missing.csv")!r})
        except lc.LightningCoreError:
            pass
        else:
            raise AssertionError("a missing file must be reported")
    """, tmp_path)


def test_attention_cache_seed_and_rows(tmp_path):
    seed = tmp_path / "attn_seed.csv"
    seed.write_text("#lc_tune_cache,attention,1\nfwd,8,8,0,0,0,0\n", encoding="utf-8")
    rows = tmp_path / "attn_rows.csv"
    rows.write_text("\n".join([
        "#lc_tune_cache,attention,2",
        "#columns,kind,seq,dim,causal,resident_hint,sync_hint,compute_loss_or_mode,mode",
        "HF,256,64,0,1,0,gfx950,4",
        "HF,2048,128,1,0,1,gfx950,2",
        "HT,256,64,1,0,1,1,gfx950,8",
        "HF,256,64,0,1,0,gfx942,2",  # another arch: its own row, not this device's
        "HF,96,48,0,0,0,gfx950,3",   # not a gfx950 split count: dropped
        "HT,96,48,0,0,0,gfx950,1",   # HT row without compute_loss: ignored
        "HF,128,32,0,0,0,gfx950,16",  # the 16-query forward kernel: kept
        "HT,128,32,0,0,0,1,gfx950,16",  # the 16-key dV kernel: kept
    ]) + "\n", encoding="utf-8")
    out1 = tmp_path / "attn_out1.csv"
    out2 = tmp_path / "attn_out2.csv"
    _run(f"""
        import lightning_core as lc
        lc.attention_tune_cache_load({str(seed)!r})
        assert lc.attention_tune_cache_size() == 0
        lc.attention_tune_cache_save({str(out1)!r})
        lc.attention_tune_cache_load({str(rows)!r})
        assert lc.attention_tune_cache_size() == 6, lc.attention_tune_cache_size()
        lc.attention_tune_cache_save({str(out2)!r})
        lc.attention_reset_tuning()
        assert lc.attention_tune_cache_size() == 0
    """, tmp_path)
    l1 = _lines(out1)
    assert l1[0] == "#lc_tune_cache,attention,2"
    assert l1[1] == "#columns,kind,seq,dim,causal,resident_hint,sync_hint,compute_loss_or_mode,mode"
    assert l1[2].startswith("#columns_hip,") and len(l1) == 3
    assert sorted(_lines(out2)[3:]) == sorted(["HF,256,64,0,1,0,gfx950,4", "HF,2048,128,1,0,1,gfx950,2",
                                               "HT,256,64,1,0,1,1,gfx950,8", "HF,256,64,0,1,0,gfx942,2",
                                               "HF,128,32,0,0,0,gfx950,16", "HT,128,32,0,0,0,1,gfx950,16"])


def test_attention_cache_keeps_reference_rows(tmp_path):
    """A file the reference wrote (Metal forward modes 1-3, train modes) is
    kept verbatim on rewrite, and none of its rows is read as a gfx950 split
    count (src/attention_metal.mm:184-336 reads only 7-column F and 8-column
    T rows, so it skips the HF / HT rows written here)."""
    ref = tmp_path / "attn_ref.csv"
    ref_rows = ["F,256,64,0,1,0,3", "F,512,64,1,0,1,1", "T,256,64,1,0,1,1,2"]
    ref.write_text("#lc_tune_cache,attention,2\n"
                   "#columns,kind,seq,dim,causal,resident_hint,sync_hint,compute_loss_or_mode,mode\n"
                   + "\n".join(ref_rows) + "\n", encoding="utf-8")
    out = tmp_path / "attn_out.csv"
    _run(f"""
        import lightning_core as lc
        lc.attention_tune_cache_load({str(ref)!r})
        assert lc.attention_tune_cache_size() == 0, lc.attention_tune_cache_size()
        lc.attention_tune_cache_save({str(out)!r})
    """, tmp_path)
    lines = _lines(out)
    assert lines[0] == "#lc_tune_cache,attention,2"
    body = [l for l in lines if not l.startswith("#")]
    assert body == ref_rows
    # the reference's row filter (exactly 7 columns for F, 8 for T) keeps only its own rows
    hip_row = "HF,256,64,0,1,0,gfx950,4"
    cols = hip_row.split(",")
    assert not ((len(cols) == 7 and cols[0] == "F") or (len(cols) == 8 and cols[0] == "T"))


_GETENV = """
    import ctypes
    libc = ctypes.CDLL(None)
    libc.getenv.restype = ctypes.c_char_p
    def cenv(k):
        v = libc.getenv(k.encode())
        return None if v is None else v.decode()
"""


def test_runtime_profile_env_file(tmp_path):
    prof = tmp_path / "profile.env"
    prof.write_text("\n".join([
        "# runtime profile",
        "CJ_TEST_ALPHA=1",
        "  CJ_TEST_BETA =  two  ",
        "OTHER_VAR=3",
        "CJ_TEST_KEEP=from_file",
        "CJ_TEST_EMPTY=",
        "=novalue",
    ]) + "\n", encoding="utf-8")
    _run(_GETENV + """
        import lightning_core as lc
        lc.preload_runtime_profile_env()
        assert cenv("CJ_TEST_ALPHA") == "1"
        assert cenv("CJ_TEST_BETA") == "two"
        assert cenv("OTHER_VAR") is None          # only CJ_* keys are imported
        assert cenv("CJ_TEST_KEEP") == "preset"   # never overrides a set variable
        assert cenv("CJ_TEST_EMPTY") is None
    """, tmp_path, {"CJ_RUNTIME_PROFILE_ENV_FILE": str(prof), "CJ_TEST_KEEP": "preset"})


def test_runtime_profile_cwd_candidate_and_autoload_off(tmp_path):
    (tmp_path / "model_runtime_profile.env").write_text("CJ_TEST_CWD=yes\n", encoding="utf-8")
    _run(_GETENV + """
        import lightning_core as lc
        lc.preload_runtime_profile_env()
        assert cenv("CJ_TEST_CWD") == "yes"
    """, tmp_path)
    _run(_GETENV + """
        import lightning_core as lc
        lc.preload_runtime_profile_env()
        assert cenv("CJ_TEST_CWD") is None
    """, tmp_path, {"CJ_RUNTIME_PROFILE_AUTOLOAD": "off"})
