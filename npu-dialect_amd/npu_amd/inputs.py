"""Seeded synthetic inputs: a counter-based SplitMix64 stream per tensor.

Element i of tensor t under seed s is ``mix64(key(s, t) + (i + 1) * GOLDEN)``
where ``mix64`` is the SplitMix64 output function (Steele, Lea & Flood 2014)
and ``key(s, t) = mix64(s ^ (t << 32))``.  Uniform draws take the top 53
bits; normal draws use Box-Muller on consecutive pairs.  Everything is
vectorised numpy uint64 arithmetic (wrapping mod 2^64), so the same seed gives
the same tensors on any host.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

SEED_BASE = 0x4E505500  # "NPU\0" + config number


def mix64(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64, copy=True)
    with np.errstate(over="ignore"):
        z ^= z >> np.uint64(30)
        z *= _M1
        z ^= z >> np.uint64(27)
        z *= _M2
        z ^= z >> np.uint64(31)
    return z


def raw(seed: int, tensor_id: int, n: int) -> np.ndarray:
    key = mix64(np.array([(seed ^ (tensor_id << 32)) & 0xFFFFFFFFFFFFFFFF], np.uint64))[0]
    with np.errstate(over="ignore"):
        ctr = key + (np.arange(1, n + 1, dtype=np.uint64) * GOLDEN)
    return mix64(ctr)


def unit(seed, tensor_id, n):
    """Uniform in [0, 1) with 53-bit resolution (float64)."""
    return (raw(seed, tensor_id, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def uniform(seed, tensor_id, shape, lo, hi) -> np.ndarray:
    n = int(np.prod(shape))
    return (lo + (hi - lo) * unit(seed, tensor_id, n)).astype(np.float32).reshape(shape)


def normal(seed, tensor_id, shape, mean=0.0, std=1.0) -> np.ndarray:
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = unit(seed, tensor_id, 2 * m)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    rad = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, np.float64)
    z[0::2] = rad * np.cos(2.0 * np.pi * u2)
    z[1::2] = rad * np.sin(2.0 * np.pi * u2)
    return (mean + std * z[:n]).astype(np.float32).reshape(shape)


def randint(seed, tensor_id, shape, lo, hi) -> np.ndarray:
    """Integers uniform in [lo, hi] (inclusive), int64."""
    n = int(np.prod(shape))
    r = raw(seed, tensor_id, n) >> np.uint64(32)
    return (lo + (r % np.uint64(hi - lo + 1)).astype(np.int64)).reshape(shape)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)
