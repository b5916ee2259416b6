"""Seeded synthetic inputs for the benchmark configurations.

SplitMix64 (Steele, Lea & Flood 2014) with seed = 0x5EED0000 + tensor_index;
u = (x >> 40) * 2^-24 in [0, 1); U(a, b) = a + (b - a) * u; N(mu, sigma) by
Box-Muller on consecutive pairs; Kaiming-uniform = U(+-sqrt(6 / fan_in)).
fp16 tensors are generated in float32 and rounded to nearest even.  The same
bits feed the HIP kernels and every CPU check.
"""
from __future__ import annotations

import numpy as np

SEED_BASE = 0x5EED0000
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    idx = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def unit(seed: int, n: int) -> np.ndarray:
    return (splitmix64(seed, n) >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)


def uniform(index: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape))
    return (lo + (hi - lo) * unit(SEED_BASE + index, n)).astype(np.float32).reshape(shape)


def normal(index: int, shape, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = unit(SEED_BASE + index, 2 * m)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mu + sigma * z[:n]).astype(np.float32).reshape(shape)


def kaiming_uniform(index: int, shape) -> np.ndarray:
    """Conv weight [OC, IC/groups, KH, KW] or linear weight: fan_in = prod(shape[1:])."""
    fan_in = int(np.prod(shape[1:]))
    b = float(np.sqrt(6.0 / fan_in))
    return uniform(index, shape, -b, b)


def ref_pattern(shape) -> np.ndarray:
    """The reference benchmark's input pattern (i % 251) / 250 - 0.5."""
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.int64)
    return ((i % 251) / 250.0 - 0.5).astype(np.float32).reshape(shape)


def as_f16(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest float16 and return it as float32."""
    return x.astype(np.float16).astype(np.float32)
