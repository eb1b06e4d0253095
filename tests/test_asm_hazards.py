"""Hardware-hazard scan of the built gfx950 kernels (CPU only: hipcc -S).

The global -> LDS copies are inline asm (kcommon.hpp, load_lds16_sbase and
its variants), and the compiler does not pad the inside of an asm statement
for hazards.  Two apply to these copies (AMD CDNA3/CDNA4 ISA, "manually
inserted wait states"):

* a VALU write of an SGPR needs 5 wait states before a VMEM instruction reads
  that SGPR.  The copy's 64-bit base may arrive straight from a v_readlane
  (a spilled SGPR reloaded by the compiler): one wait state after it, a copy
  took a stale half of its base and faulted the GPU.  The asm therefore reads
  an SALU copy of the base made by its first instruction, or (several copies
  of one part) an SALU copy made by the first copy's asm earlier in the same
  basic block;
* an SALU write of M0 needs 1 wait state before an LDS-DMA load reads M0
  (the SALU copy above is that wait state for a part's first copy; later
  copies reuse M0); a VALU write of M0 would need 5.

The scan applies the rules themselves: for every LDS-DMA load, each SGPR of
its base pair must have been last written, in the same basic block, by an
SALU instruction, and no VALU write of it may lie within 5 wait states; the
instruction right before the load must not write M0, and no VALU writes M0.

A third check covers a second fault of the same family, in host-visible
kernel code rather than the asm: a 64-bit base rebuilt from a 32-bit
v_readfirstlane result, whose high half then came from sign-extending the low
half (s_ashr_i32 hi, lo, 31) instead of from the pointer.  The scan traces
each copy's base pair back to its last writers and flags that shape.

The scan checks every LDS-DMA load in the compiled kernels, and planted
instances of the faulting sequences show the scan catches them.  The same
compile also checks that no kernel spills to scratch (a nonzero private
segment in its descriptor).
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


def _dest(t):
    """SGPRs an instruction writes (its first operand), for s_* and v_* ops."""
    parts = t.split(None, 1)
    if len(parts) < 2 or not (parts[0].startswith("s_") or parts[0].startswith("v_")):
        return set()
    return _sregs(parts[1].split(",")[0])


def _last_writer(ins, i, reg):
    """Index of the last instruction before i that writes `reg` (None at a
    label: a control-flow merge ends the straight-line trace)."""
    for j in range(i - 1, -1, -1):
        if ins[j].endswith(":"):
            return None
        if reg in _dest(ins[j]):
            return j
    return None


def _sign_extended_readfirstlane_base(ins, i, pair):
    """The copy at i reads `pair`: is its high half s_ashr_i32 of its low
    half, with the low half written by v_readfirstlane?"""
    m = re.match(r"s\[(\d+):(\d+)\]$", pair)
    if not m:
        return False
    lo, hi = f"s{m.group(1)}", f"s{m.group(2)}"
    j = _last_writer(ins, i, hi)
    if j is None or not re.match(rf"^s_ashr_i32\s+{hi},\s*{lo},\s*31$", ins[j]):
        return False
    k = _last_writer(ins, j, lo)
    return k is not None and ins[k].startswith("v_readfirstlane_b32")


def _wait_states(t):
    """Wait states an instruction provides (s_nop N: N + 1)."""
    m = re.match(r"^s_nop\s+(\d+)", t)
    return int(m.group(1)) + 1 if m else 1


def scan(text):
    """Problems found: LDS-DMA loads whose SGPR base was last written by a
    VALU instruction (or by anything outside the load's basic block), VALU
    writes of a base SGPR within 5 wait states of a load, M0 written by the
    instruction right before a load, VALU writes of M0, and bases whose high
    half is a sign-extended v_readfirstlane result."""
    problems = []
    ins = _instructions(text)
    for i, t in enumerate(ins):
        if re.match(r"^v_\w+\s+m0\b", t):
            problems.append(f"VALU writes M0: {t}")
        m = _LOAD.match(t)
        if not m:
            continue
        base = m.group(1)
        if i > 0 and "m0" in _dest(ins[i - 1]):
            problems.append(f"M0 written with no wait state before the load: [{ins[i - 1]}] -> [{t}]")
        # the last writer of each half, in this basic block, is an SALU
        # instruction (a VALU one is also reported when it lies within 5 wait
        # states, the faulting case)
        writers = set()
        for reg in sorted(_sregs(base)):
            j = _last_writer(ins, i, reg)
            if j is None:
                problems.append(f"load base {reg} not written in the load's basic block: [{t}]")
            elif not ins[j].startswith("s_"):
                ws = sum(_wait_states(x) for x in ins[j + 1:i])
                if ws < 5:
                    problems.append(f"VALU write of {reg} {ws} wait states before the load: [{ins[j]}] -> [{t}]")
                problems.append(f"load base {reg} last written by a non-SALU instruction: [{ins[j]}] -> [{t}]")
            else:
                writers.add(j)
        # a base copied by s_mov_b64: check where the copy came from
        if len(writers) == 1:
            j = writers.pop()
            pm = re.match(r"^s_mov_b64\s+(s\[\d+:\d+\]),\s*(s\[\d+:\d+\])$", ins[j])
            src, at = (pm.group(2), j) if pm and pm.group(1) == base else (base, i)
        else:
            src, at = base, i
        if _sign_extended_readfirstlane_base(ins, at, src):
            problems.append(f"load base {src} is a sign-extended v_readfirstlane value: [{t}]")
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
    found = scan(planted)
    assert any("VALU write of s7 1 wait states" in f for f in found), found
    fixed = planted.replace("s_nop 0", "s_mov_b64 s[40:41], s[6:7]").replace("v195, s[6:7]", "v195, s[40:41]")
    assert scan(fixed) == []
    assert scan("\tv_readfirstlane_b32 m0, v3\n") != []


def test_scan_accepts_a_shared_salu_copy_and_catches_a_bare_m0_write():
    # the copies of one part: the first asm copies the base, the next read the copy
    shared = "\n".join([
        "\ts_add_u32 s2, s4, s33",
        "\ts_addc_u32 s3, s5, s34",
        "\ts_mov_b32 m0, s27",
        "\ts_mov_b64 s[36:37], s[2:3]",
        "\tglobal_load_lds_dwordx4 v64, s[36:37]",
        "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]",
        "\tglobal_load_lds_dwordx4 v68, s[36:37] offset:1024",
        "\tds_read_b128 v[8:11], v85 offset:2048",
        "\tglobal_load_lds_dwordx4 v72, s[36:37] offset:2048",
    ])
    assert scan(shared) == []
    # M0 rewritten right before a later copy: no wait state
    bare_m0 = shared.replace("\tglobal_load_lds_dwordx4 v72", "\ts_mov_b32 m0, s28\n\tglobal_load_lds_dwordx4 v72")
    found = scan(bare_m0)
    assert len(found) == 1 and "M0" in found[0], found
    # the shared copy reloaded by the compiler between the copies (a spill)
    reload = shared.replace("\tds_read_b128 v[8:11], v85 offset:2048",
                            "\tv_readlane_b32 s36, v200, 3\n\ts_nop 1")
    found = scan(reload)
    assert any("VALU write" in f for f in found) and any("non-SALU" in f for f in found), found
    # ... or a base that reaches the copy across a label
    merged = shared.replace("\tv_mfma_f32_16x16x32_bf16", ".LBB0_7:\n\tv_mfma_f32_16x16x32_bf16")
    found = scan(merged)
    assert len(found) == 4 and all("basic block" in f for f in found), found  # two loads, two halves each


def test_scan_catches_a_sign_extended_readfirstlane_base():
    planted = "\n".join([
        "\tv_readfirstlane_b32 s10, v5",
        "\ts_ashr_i32 s11, s10, 31",
        "\ts_mov_b32 m0, s3",
        "\t;;#ASMSTART",
        "\ts_mov_b64 s[40:41], s[10:11]",
        "\tglobal_load_lds_dwordx4 v1, s[40:41] offset:1024",
        "\t;;#ASMEND",
    ])
    found = scan(planted)
    assert len(found) == 1 and "sign-extended" in found[0], found
    # a base built by 64-bit adds from the kernel argument is fine, and so is
    # a sign-extended 32-bit offset that is added to the base
    fixed = "\n".join([
        "\tv_readfirstlane_b32 s10, v5",
        "\ts_ashr_i32 s11, s10, 31",
        "\ts_lshl_b64 s[10:11], s[10:11], 1",
        "\ts_add_u32 s12, s4, s10",
        "\ts_addc_u32 s13, s5, s11",
        "\ts_mov_b32 m0, s3",
        "\ts_mov_b64 s[40:41], s[12:13]",
        "\tglobal_load_lds_dwordx4 v1, s[40:41]",
    ])
    assert scan(fixed) == []


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
    spills = []
    kernels = 0
    for out in outs:
        for name, desc in re.findall(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", open(out).read(), re.S):
            kernels += 1
            m = re.search(r"\.amdhsa_private_segment_fixed_size (\d+)", desc)
            if m is None or int(m.group(1)) > 0:
                spills.append(f"{os.path.basename(out)}: {name} private segment {m.group(1) if m else '?'} bytes")
    assert kernels > 0, "no kernel descriptors found"
    assert not spills, "\n".join(spills[:20])
