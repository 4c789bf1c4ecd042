"""The benchmark configurations' synthetic inputs, generated in HBM from the portable RNG.

Config 1 (isolated fp32 time self-attention): B=256 series, L=513 tokens (512 context patches of
an 8192-step context plus [REG]), 12 heads x 64, d_model 768. x ~ N(0,1) [B*L, 768] and
Wqkv ~ N(0, 0.02) [2304, 768]; qkv = x Wqkv^T in fp32. Per-series left padding U{0..256}
context tokens is dead (live = 0); [REG] is always live. RoPE base 1e4 at the token index.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import rng
from .chronos2 import rope_table
from .runtime import fill_normal


@dataclass
class TimeCase:
    rows: int
    n: int
    heads: int
    dh: int
    inner: int
    qkv: object  # torch [rows*n, 3*inner]
    live: object  # torch int32 [rows*n]
    table: object  # torch float32 [n, dh]
    pads: np.ndarray

    def mask_aware_flops(self) -> float:
        """sum over (row, head, query) of 4*dh*|live keys of the row| (QK^T and PV only)."""
        live_per_row = self.live.view(self.rows, self.n).sum(dim=1).double().sum().item()
        return 4.0 * self.dh * self.heads * self.n * live_per_row

    def dense_flops(self) -> float:
        return 4.0 * self.dh * self.n * self.n * self.heads * self.rows


def c2_time_config1(rows: int = 256, n: int = 513, heads: int = 12, dh: int = 64, d_model: int = 768,
                    max_pad: int = 256, seed: int = 0, device: str = "cuda") -> TimeCase:
    import torch

    inner = heads * dh
    x = torch.empty(rows * n, d_model, dtype=torch.float32, device=device)
    w = torch.empty(3 * inner, d_model, dtype=torch.float32, device=device)
    fill_normal(x, rng.stream_seed(seed, 0), 0.0, 1.0)
    fill_normal(w, rng.stream_seed(seed, 1), 0.0, 0.02)
    qkv = x @ w.t()
    del x
    pads = rng.randint(rng.stream_seed(seed, 2), rows, 0, max_pad)
    t = np.arange(n)[None, :]
    live = (t >= pads[:, None]).astype(np.int32)
    live[:, n - 1] = 1  # [REG]
    live_t = torch.from_numpy(live.reshape(-1)).to(device)
    table = torch.from_numpy(rope_table(n, dh)).to(device)
    return TimeCase(rows, n, heads, dh, inner, qkv.contiguous(), live_t, table, pads)


@dataclass
class GroupCase:
    rows: int
    n: int
    heads: int
    dh: int
    inner: int
    qkv: object  # torch [rows*n, 3*inner]
    live: object  # torch int32 [rows*n]
    group_start: object  # torch int32 [rows]
    group_end: object
    group: np.ndarray

    def algorithmic_bytes(self) -> float:
        """Read q, k, v once and write out once, fp32: rows*n*(3*inner + inner)*4."""
        return float(self.rows) * self.n * 4 * self.inner * 4

    def flops(self) -> float:
        """QK^T and PV over the (live) same-group pairs of every slot: 4*dh per pair per head."""
        sizes = np.bincount(self.group)
        live_slots = self.live.view(self.rows, self.n).sum().item() / self.rows  # all live in config 2
        return 4.0 * self.dh * self.heads * float((sizes.astype(np.float64) ** 2).sum()) * live_slots


def c2_group_config2(rows: int = 4096, n: int = 129, heads: int = 12, dh: int = 64, lo: int = 1, hi: int = 64,
                     seed: int = 0, device: str = "cuda") -> GroupCase:
    """Config 2: qkv ~ N(0,1) [rows*n, 3*inner]; contiguous groups with sizes U{lo..hi} (the last
    truncated); every slot live."""
    import torch

    from .chronos2 import group_bounds

    inner = heads * dh
    qkv = torch.empty(rows * n, 3 * inner, dtype=torch.float32, device=device)
    fill_normal(qkv, rng.stream_seed(seed, 0), 0.0, 1.0)
    sizes = rng.randint(rng.stream_seed(seed, 3), rows, lo, hi)
    group = np.repeat(np.arange(rows, dtype=np.int32), sizes)[:rows]
    s, e = group_bounds(group)
    live = torch.ones(rows * n, dtype=torch.int32, device=device)
    return GroupCase(rows, n, heads, dh, inner, qkv, live, torch.from_numpy(s).to(device),
                     torch.from_numpy(e).to(device), group)
