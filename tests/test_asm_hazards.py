"""Hardware-hazard scan of the built gfx950 kernels (CPU only: hipcc -S).

The global -> LDS copies are inline asm (kcommon.hpp, load_lds16_sbase), and
the compiler does not pad the inside of an asm statement for hazards.  Two
apply to these copies (AMD CDNA3/CDNA4 ISA, "manually inserted wait states"):

* a VALU write of an SGPR needs 5 wait states before a VMEM instruction reads
  that SGPR.  The copy's 64-bit base may arrive straight from a v_readlane
  (a spilled SGPR reloaded by the compiler): one wait state after it, a copy
  took a stale half of its base and faulted the GPU.  The asm therefore reads
  an SALU copy of the base made by its first instruction;
* an SALU write of M0 needs 1 wait state before an LDS-DMA load reads M0
  (the SALU copy above is that wait state); a VALU write of M0 would need 5.

The scan checks every LDS-DMA load in the compiled kernels for both, and a
planted instance of the faulting sequence shows the scan catches it.
"""
import concurrent.futures
import glob
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "lightining-core_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

_LOAD = re.compile(r"^\s*global_load_lds_dwordx4\s+v\d+,\s*(s\[\d+:\d+\])")


def _sregs(tok):
    tok = tok.strip().rstrip(",")
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    if re.match(r"s\d+$", tok) or tok == "m0":
        return {tok}
    return set()


def _instructions(text):
    """Instruction lines (comments, directives and asm markers dropped)."""
    out = []
    for line in text.split("\n"):
        t = line.split(";")[0].strip()
        if not t or (t.startswith(".") and not t.endswith(":")):
            continue
        out.append(t)
    return out


def scan(text):
    """Problems found: LDS-DMA loads whose SGPR base is not an SALU copy made
    by the instruction right before, and VALU writes of M0."""
    problems = []
    ins = _instructions(text)
    for i, t in enumerate(ins):
        if re.match(r"^v_\w+\s+m0\b", t):
            problems.append(f"VALU writes M0: {t}")
        m = _LOAD.match(t)
        if not m:
            continue
        base = m.group(1)
        prev = ins[i - 1] if i > 0 else ""
        pm = re.match(r"^s_mov_b64\s+(s\[\d+:\d+\]),", prev)
        if not pm or pm.group(1) != base:
            problems.append(f"load reads {base} not copied by the previous SALU move: [{prev}] -> [{t}]")
    return problems


def _compile_asm(src, out_dir):
    out = os.path.join(out_dir, os.path.basename(src) + ".s")
    cmd = [HIPCC, "-x", "hip", "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC, "--cuda-device-only",
           "-S", src, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out


def test_scan_catches_the_faulting_sequence():
    planted = "\n".join([
        "\tv_readlane_b32 s6, v219, 16",
        "\ts_mov_b32 m0, s92",
        "\tv_readlane_b32 s7, v219, 17",
        "\t;;#ASMSTART",
        "\ts_nop 0",
        "\tglobal_load_lds_dwordx4 v195, s[6:7]",
        "\t;;#ASMEND",
    ])
    assert len(scan(planted)) == 1
    fixed = planted.replace("s_nop 0", "s_mov_b64 s[40:41], s[6:7]").replace("v195, s[6:7]", "v195, s[40:41]")
    assert scan(fixed) == []
    assert scan("\tv_readfirstlane_b32 m0, v3\n") != []


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
def test_built_kernels_have_no_lds_dma_hazards(tmp_path):
    srcs = sorted(glob.glob(os.path.join(CSRC, "kernels", "*.hip")))
    assert srcs
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(4, len(srcs))) as ex:
        outs = list(ex.map(lambda s: _compile_asm(s, str(tmp_path)), srcs))
    loads = 0
    problems = []
    for out in outs:
        text = open(out).read()
        loads += sum(1 for t in _instructions(text) if _LOAD.match(t))
        problems += [f"{os.path.basename(out)}: {p}" for p in scan(text)]
    assert loads > 0, "no LDS-DMA loads found: the scan pattern no longer matches the kernels"
    assert not problems, "\n".join(problems[:20])
