"""Shared helpers for the GPU parity tests.

Tolerances (north star): normwise max|d| / max|ref| <= 1e-4 for fp32 and
<= 2e-2 for bf16 / fp16 with fp32 accumulate, where the CPU oracle runs on the
inputs rounded to the compute dtype and promoted back to fp32.
"""
import sys

import numpy as np
import pytest

import oracle_lib

TOL = {"f32": 1e-4, "bf16": 2e-2, "f16": 2e-2}


def require_hip():
    import lightning_core as lc

    if not lc.is_hip_available():
        pytest.fail("no gfx950 HIP device visible: GPU tests must run on an MI355X (no fallback exists)")
    return lc


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def assert_parity(ref, got, dtype, what=""):
    err = oracle_lib.normwise_rel(ref, got)
    note(f"[parity] {what} dtype={dtype} normwise_rel={err:.3e} tol={TOL[dtype]:.0e}")
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert err <= TOL[dtype], f"{what}: normwise relative error {err:.3e} > {TOL[dtype]:.0e}"
    return err
