"""Seeded synthetic inputs for the benchmark configurations.

SplitMix64 (Steele, Lea & Flood, "Fast splittable pseudorandom number
generators", OOPSLA 2014) → top 24 bits → U[0,1); normals by the
Box–Muller transform.  One stream per tensor, seeded 1000·config + tensor
index, so the GPU run and the CPU baseline see identical bits.
`normal(n, seed, var)` takes the variance (N(0, 2/fan_in) etc.).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(n: int, seed: int) -> np.ndarray:
    """The first n outputs of SplitMix64 started at `seed`."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + _GOLDEN * np.arange(1, n + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform01(n: int, seed: int) -> np.ndarray:
    """U[0,1) with 24-bit resolution, float64."""
    return (splitmix64(n, seed) >> np.uint64(40)).astype(np.float64) / float(1 << 24)


def uniform(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    return (lo + (hi - lo) * uniform01(n, seed)).astype(np.float32)


def normal(n: int, seed: int, var: float = 1.0) -> np.ndarray:
    """N(0, var) as float32 (Box–Muller on consecutive pairs)."""
    m = (n + 1) // 2
    u = uniform01(2 * m, seed)
    u1, u2 = 1.0 - u[0::2], u[1::2]  # u1 in (0, 1]
    r = np.sqrt(-2.0 * np.log(u1)) * np.sqrt(var)
    out = np.empty(2 * m, np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return out[:n].astype(np.float32)
