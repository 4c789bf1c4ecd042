"""Seeded synthetic inputs for the parity tests (the portable RNG of jitcast_amd.rng)."""
from __future__ import annotations

import numpy as np

from jitcast_amd import rng


def qkv(seed: int, tokens: int, inner: int, std: float = 1.0) -> np.ndarray:
    return rng.normal(rng.stream_seed(seed, 0), tokens * 3 * inner, std).reshape(tokens, 3 * inner)


def left_pad_live(seed: int, rows: int, n: int, max_pad: int, tail_live: int = 1) -> np.ndarray:
    """live[r, t] = t >= pad_r for the context tokens, the last `tail_live` tokens always live."""
    pads = rng.randint(rng.stream_seed(seed, 1), rows, 0, max_pad)
    t = np.arange(n)[None, :]
    live = (t >= pads[:, None]).astype(np.int32)
    if tail_live:
        live[:, n - tail_live:] = 1
    return live


def random_live(seed: int, rows: int, n: int, p: float) -> np.ndarray:
    return (rng.uniform(rng.stream_seed(seed, 2), rows * n) < p).astype(np.int32).reshape(rows, n)


def group_sizes(seed: int, rows: int, lo: int, hi: int) -> np.ndarray:
    """Group ids of contiguous runs with sizes uniform in [lo, hi] (the last truncated)."""
    sizes = rng.randint(rng.stream_seed(seed, 3), rows, lo, hi)
    ids = np.empty(rows, np.int32)
    r = g = 0
    for s in sizes:
        if r >= rows:
            break
        e = min(rows, r + int(s))
        ids[r:e] = g
        r, g = e, g + 1
    return ids
