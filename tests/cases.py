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


def ts_layout(seed: int, rows: int, enc: int, ll: int, h: int, known_frac: float = 0.0, max_start: int | None = None):
    """A Timestral block layout in the shape BlockLayout.of produces (BlockLayout.java:77-148):
    each row starts observing at patch s_r (attend_missing_patches: every patch from s_r on is a
    valid key), rows are known covariates with probability known_frac, positions count patches from
    the row's first observed patch (decoder tokens continue from ll). Returns (key_valid [rows, enc],
    known [rows], position [rows, enc + h]) int32; the table row of a token is position + enc."""
    ms = enc // 2 if max_start is None else max_start
    starts = rng.randint(rng.stream_seed(seed, 4), rows, 0, ms)
    k = np.arange(enc)[None, :]
    key_valid = (k >= starts[:, None]).astype(np.int32)
    known = (rng.uniform(rng.stream_seed(seed, 5), rows) < known_frac).astype(np.int32)
    n = enc + h
    t = np.arange(n)[None, :]
    raw = np.where(t < enc, t, ll + t - enc)
    first = np.where(starts < enc, starts, 0)
    position = (raw - first[:, None]).astype(np.int32)
    return key_valid, known, position
