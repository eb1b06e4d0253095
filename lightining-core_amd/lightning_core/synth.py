"""Seeded synthetic inputs shared by the benchmark and the parity tests.

Both the HIP path and the CPU checker consume the same bytes: values are
generated in float64 from a SplitMix64 stream, cast to float32, and (for the
half-precision configurations) rounded to bfloat16 / float16 with
round-to-nearest-even; the checker then runs on the rounded values promoted
back to float32, so parity measures only the GPU arithmetic.

`make_value` restates the reference's deterministic test generator
(tests/test_backend_parity.cpp:12-23).
"""
from __future__ import annotations

import numpy as np

DEFAULT_SEED = 20260401  # benchmarks/python/quick_bench.py:166 default seed

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 23


def _splitmix64(seed: int, start: int, count: int) -> np.ndarray:
    """Outputs start..start+count-1 of the SplitMix64 stream seeded with `seed`."""
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _unit(bits: np.ndarray) -> np.ndarray:
    """Uniform float64 in [0, 1) from the top 53 bits."""
    return (bits >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def uniform(shape, seed: int = DEFAULT_SEED, lo: float = -1.0, hi: float = 1.0, stream: int = 0) -> np.ndarray:
    """float32 array of U(lo, hi) values; `stream` selects an independent stream."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    base = seed * 1000003 + stream
    for s in range(0, n, _CHUNK):
        c = min(_CHUNK, n - s)
        u = _unit(_splitmix64(base, s, c))
        out[s:s + c] = (lo + (hi - lo) * u).astype(np.float32)
    return out.reshape(shape)


def normal(shape, seed: int = DEFAULT_SEED, std: float = 1.0, stream: int = 0) -> np.ndarray:
    """float32 array of N(0, std^2) values (Box-Muller over pairs of uniforms)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    base = seed * 1000003 + stream
    pairs = (n + 1) // 2
    for s in range(0, pairs, _CHUNK):
        c = min(_CHUNK, pairs - s)
        bits = _splitmix64(base, 2 * s, 2 * c)
        u1 = 1.0 - _unit(bits[0::2])  # (0, 1]
        u2 = _unit(bits[1::2])
        r = np.sqrt(-2.0 * np.log(u1)) * std
        th = 2.0 * np.pi * u2
        vals = np.empty(2 * c, dtype=np.float64)
        vals[0::2] = r * np.cos(th)
        vals[1::2] = r * np.sin(th)
        lo = 2 * s
        hi = min(n, lo + 2 * c)
        out[lo:hi] = vals[: hi - lo].astype(np.float32)
    return out.reshape(shape)


def make_value(i, scale: float = 1.0) -> np.ndarray:
    """tests/test_backend_parity.cpp:12-15: ((i*37 + 11) mod 97 - 48) * scale."""
    i = np.asarray(i, dtype=np.uint64)
    v = ((i * np.uint64(37) + np.uint64(11)) % np.uint64(97)).astype(np.int64) - 48
    return v.astype(np.float32) * np.float32(scale)


def make_vec(n: int, scale: float = 0.01, bias: float = 0.0) -> np.ndarray:
    """tests/test_backend_parity.cpp:17-23 (makeVec)."""
    return (make_value(np.arange(n), scale) + np.float32(bias)).astype(np.float32)


# --- half-precision rounding (round to nearest, ties to even) ---------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), RNE; NaN stays NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = ((u >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
    with np.errstate(over="ignore"):
        r = ((u + rounding) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = r.copy()
        r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (returned as float32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x)).reshape(np.shape(x))


def round_f16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest float16 (returned as float32)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return round_f16(x)
    raise ValueError(f"unknown dtype {dtype!r}")
