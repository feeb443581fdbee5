"""Deterministic synthetic inputs for the benchmark configurations.

One counter-based generator (splitmix64 finaliser over seed/stream/counter),
written with numpy uint64 arithmetic only, so every platform produces the same
bytes; no numpy.random, no libm.  Distributions follow the benchmark configs:

  sign bits        Bernoulli(0.5): uniform random bytes
  fp16 scales      U[lo, hi) in float64, rounded to binary16 (round-to-nearest-even)
  int8 activations U[-127, 127]
  f32 activations  approx N(0, 1) by Irwin-Hall(12) from 24-bit integers (exact in
                   float64), times 20 with probability 0.001 (outliers), rounded to f32

All arithmetic before the final float rounding is exact, so the float results
are reproducible bit for bit.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def u64(seed: int, stream: int, count: int) -> np.ndarray:
    """`count` uniform uint64 values of (seed, stream)."""
    with np.errstate(over="ignore"):
        key = _mix(np.array([(seed * 0x100000001B3 + stream * 0xD6E8FEB86659FD93) & (2**64 - 1)],
                            dtype=np.uint64))[0]
        ctr = np.arange(1, count + 1, dtype=np.uint64)
        return _mix(key + ctr * _GOLDEN)


def sign_bits(n: int, k: int, seed: int, stream: int = 0) -> np.ndarray:
    """[n][k/8] uint8, LSB-first sign bits (bit 1 = +1)."""
    nbytes = n * (k // 8)
    words = u64(seed, 1000 + stream, (nbytes + 7) // 8)
    return words.view(np.uint8)[:nbytes].reshape(n, k // 8).copy()


def scales_fp16(n: int, groups: int, seed: int, lo: float = 0.01, hi: float = 0.1,
                stream: int = 0) -> np.ndarray:
    """[n][groups] uint16 binary16 bit patterns of U[lo, hi)."""
    u = (u64(seed, 2000 + stream, n * groups) >> np.uint64(11)).astype(np.float64) * 2.0**-53
    v = lo + (hi - lo) * u
    return v.astype(np.float16).view(np.uint16).reshape(n, groups)


def int8_uniform(rows: int, k: int, seed: int, stream: int = 0) -> np.ndarray:
    """[rows][k] int8 in [-127, 127]."""
    w = u64(seed, 3000 + stream, rows * k)
    return ((w % np.uint64(255)).astype(np.int64) - 127).astype(np.int8).reshape(rows, k)


def normal_f32(rows: int, k: int, seed: int, outlier_p: float = 0.001, outlier_scale: float = 20.0,
               stream: int = 0) -> np.ndarray:
    """[rows][k] float32, Irwin-Hall(12) approximation of N(0,1) with outliers."""
    count = rows * k
    w = u64(seed, 4000 + stream, 6 * count).reshape(count, 6)
    mask24 = np.uint64(0xFFFFFF)
    lo = (w & mask24).astype(np.int64)
    hi = ((w >> np.uint64(24)) & mask24).astype(np.int64)
    s = lo.sum(axis=1) + hi.sum(axis=1)  # < 12 * 2^24: exact
    x = s.astype(np.float64) * 2.0**-24 - 6.0
    threshold = np.uint64(int(outlier_p * 2.0**64))
    out = u64(seed, 5000 + stream, count) < threshold
    x = np.where(out, x * outlier_scale, x)
    return x.astype(np.float32).reshape(rows, k)


def matrix(n: int, k: int, seed: int, stream: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Random sign bits and U[0.01, 0.1) scales for an [n][k] matrix."""
    return sign_bits(n, k, seed, stream), scales_fp16(n, k // 128, seed, stream=stream)
