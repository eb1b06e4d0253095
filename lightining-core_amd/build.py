"""Builds liblightning_core_hip.so in-tree (hipcc, gfx950 only).

Usage: python lightining-core_amd/build.py
Every source is compiled as HIP for gfx950 with packed-fp32 instruction
selection disabled, then linked into one shared library next to this file.
"""
from __future__ import annotations

import concurrent.futures
import glob
import os
import subprocess
import sysconfig
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liblightning_core_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

CFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
    "-I" + CSRC,
]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.cpp")) + glob.glob(os.path.join(CSRC, "kernels", "*.hip")))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.relpath(src, CSRC).replace(os.sep, "_") + ".o")
    cmd = [HIPCC, "-x", "hip"] + CFLAGS + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{err}")
    # Inline asm must never clobber a register the compiler reserves (M0,
    # EXEC, VCC, ...): the compiler neither saves nor restores it, so a live
    # value it keeps there would be silently corrupted.  Such registers are
    # passed as operands ("{m0}") instead; the warning is a build error here.
    if "Reserved registers on the clobber list" in err:
        raise RuntimeError(f"inline asm clobbers a reserved register: {src}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


ADDR_SRC = os.path.join(CSRC, "pyaddr.c")
ADDR_LIB = os.path.join(HERE, "lightning_core", "_addr.so")


def build_addr() -> str:
    """The binding's buffer-address helper (a CPython extension, host only)."""
    inc = sysconfig.get_paths()["include"]
    tmp = ADDR_LIB + ".tmp"
    cmd = ["gcc", "-O2", "-shared", "-fPIC", "-I" + inc, ADDR_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("pyaddr build failed\n" + r.stdout + r.stderr)
    os.replace(tmp, ADDR_LIB)
    return ADDR_LIB


def build(jobs: int | None = None) -> str:
    build_addr()
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources()))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
