"""The portable seeded RNG all inputs come from, identical in every language of this build.

SplitMix64 (Steele, Lea and Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014;
constants as in Vigna's public-domain splitmix64.c): output i (i >= 1) of stream s is
mix(s + i * 0x9E3779B97F4A7C15). A uniform in [0, 1) is the top 24 bits times 2^-24; normals come
in pairs from two uniforms by Box-Muller in double, then round to float32. Tensor k of a case
seeded `seed` uses stream `seed * 1000003 + k`.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def stream_seed(seed: int, index: int) -> int:
    return (seed * 1000003 + index) & 0xFFFFFFFFFFFFFFFF


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * M1
    z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def raw64(stream: int, count: int, start: int = 0) -> np.ndarray:
    """Outputs start+1 .. start+count of the stream, as uint64."""
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(np.uint64(stream) + i * GAMMA)


def uniform(stream: int, count: int, start: int = 0) -> np.ndarray:
    """float64 uniforms in [0, 1) with 24-bit resolution."""
    return (raw64(stream, count, start) >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))


def normal(stream: int, count: int, std: float = 1.0, mean: float = 0.0, chunk: int = 1 << 24) -> np.ndarray:
    """float32 N(mean, std^2) samples, Box-Muller pairs in double."""
    out = np.empty(count, dtype=np.float32)
    pairs = (count + 1) // 2
    for p0 in range(0, pairs, chunk):
        p1 = min(pairs, p0 + chunk)
        u = uniform(stream, 2 * (p1 - p0), 2 * p0)
        u1, u2 = u[0::2], u[1::2]
        rad = np.sqrt(-2.0 * np.log(1.0 - u1))
        z = np.empty(2 * (p1 - p0), dtype=np.float64)
        z[0::2] = rad * np.cos(2.0 * np.pi * u2)
        z[1::2] = rad * np.sin(2.0 * np.pi * u2)
        z = mean + std * z
        lo, hi = 2 * p0, min(count, 2 * p1)
        out[lo:hi] = z[: hi - lo].astype(np.float32)
    return out


def uniform_range(stream: int, count: int, lo: float, hi: float) -> np.ndarray:
    return lo + (hi - lo) * uniform(stream, count)


def randint(stream: int, count: int, lo: int, hi: int) -> np.ndarray:
    """Integers uniform in [lo, hi] inclusive."""
    return lo + np.floor(uniform(stream, count) * (hi - lo + 1)).astype(np.int64)
