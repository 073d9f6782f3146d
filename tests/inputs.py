"""Seeded synthetic inputs, identical on every machine and numpy version.

splitmix64 gives the bits; uniforms take the top 24 bits of each word;
normals use Box-Muller in float64, cast to float32 once. Written with numpy
integer arithmetic only, so golden fixtures made from these inputs stay valid
across numpy releases (whose Generator distributions may change).
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _splitmix64(seed: int, count: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        idx = np.arange(1, count + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def _unit(seed: int, count: int) -> np.ndarray:
    """Uniform in (0, 1) as float64 with 24 random bits: (u + 0.5) / 2^24."""
    bits = _splitmix64(seed, count) >> np.uint64(40)
    return (bits.astype(np.float64) + 0.5) / float(1 << 24)


def uniform(shape, lo: float, hi: float, seed: int) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    u = _unit(seed, n)
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal(shape, std: float, seed: int) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    half = (n + 1) // 2
    u1 = _unit(seed, half)
    u2 = _unit(seed ^ 0x5DEECE66D, half)
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    z = np.concatenate([r * np.cos(t), r * np.sin(t)])[:n]
    return (std * z).astype(np.float32).reshape(shape)
