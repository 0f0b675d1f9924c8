"""Seeded synthetic inputs for the verify-step configurations (no randomness on the device).

Stream: SplitMix64 over a per-field counter -> 53-bit uniform doubles -> Box-Muller normals in
double -> scaled -> rounded to BF16 with round-to-nearest-even. Seeds are derived from
(config id, field tag, layer, sequence) so every tensor is independently reproducible.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(x: np.ndarray) -> np.ndarray:
    """Vectorized SplitMix64 finalizer applied to x + golden (public algorithm)."""
    with np.errstate(over="ignore"):
        z = (x + _GOLDEN).astype(np.uint64)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def derive_seed(*parts: int) -> int:
    h = np.uint64(0x243F6A8885A308D3)
    for p in parts:
        h = splitmix64(np.array([h ^ np.uint64(p & 0xFFFFFFFFFFFFFFFF)], dtype=np.uint64))[0]
    return int(h)


def uniforms(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n doubles in [0, 1) from SplitMix64(seed + golden * (i + offset))."""
    with np.errstate(over="ignore"):
        i = np.arange(offset, offset + n, dtype=np.uint64)
        x = np.uint64(seed) + i * _GOLDEN
        return (splitmix64(x) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normals(seed: int, n: int) -> np.ndarray:
    """n standard normals (Box-Muller in double over pairs of uniforms)."""
    m = (n + 1) // 2
    u = uniforms(seed, 2 * m)
    u1 = np.maximum(u[0::2], 1e-300)
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:n]


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even FP32 -> BF16 bit patterns (uint16)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (b & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    lsb = (b >> np.uint64(16)) & np.uint64(1)
    r = ((b + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    r[nan] = ((b[nan] >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(seed: int, n: int, std: float = 1.0) -> np.ndarray:
    return f32_to_bf16_bits((normals(seed, n) * std).astype(np.float32))


def uniform_bf16(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    """n values uniform in [lo, hi), rounded to BF16."""
    return f32_to_bf16_bits((lo + (hi - lo) * uniforms(seed, n)).astype(np.float32))


def normal_bf16_with_outliers(seed: int, n: int, frac: float = 0.01, value: float = 20.0) -> np.ndarray:
    """N(0,1) with a seeded `frac` of entries replaced by +-value (long-context config)."""
    x = normals(seed, n).astype(np.float32)
    u = uniforms(seed ^ 0x5A5A5A5A, n)
    sel = u < frac
    sign = np.where(uniforms(seed ^ 0x3C3C3C3C, n) < 0.5, -1.0, 1.0).astype(np.float32)
    x[sel] = sign[sel] * np.float32(value)
    return f32_to_bf16_bits(x)


def int_uniform(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Integers uniform in [lo, hi)."""
    return (lo + np.floor(uniforms(seed, n) * (hi - lo))).astype(np.int64)
