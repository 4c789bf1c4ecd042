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


@dataclass
class LayerCase:
    rows: int
    n: int
    heads: int
    dh: int
    d: int
    dff: int
    groups: int
    x: object  # torch [rows*n, d]
    weights: dict  # torch tensors keyed like jc_c2_layer_weights
    live: object  # torch int32 [rows*n]
    table: object  # torch float32 [n, dh]
    group_start: object  # torch int32 [rows]
    group_end: object
    workspace: object  # torch float32, jc_c2_layer_workspace_bytes

    def gemm_flops(self) -> float:
        t, d, inner = self.rows * self.n, self.d, self.heads * self.dh
        return 2.0 * t * d * (2 * 3 * inner + 2 * inner + 2 * self.dff)

    def attention_flops(self) -> float:
        """time attention over every (live) key of the row, group attention over the group's rows."""
        per_group = self.rows // self.groups
        live = float(self.live.double().sum().item())
        return 4.0 * self.dh * self.heads * (self.n * live + per_group * live)

    def flops(self) -> float:
        return self.gemm_flops() + self.attention_flops()


def c2_layer_config4(groups: int = 1024, per_group: int = 5, nc: int = 128, h: int = 4, heads: int = 12, dh: int = 64,
                     d: int = 768, dff: int = 3072, seed: int = 0, device: str = "cuda") -> LayerCase:
    """Config 4's encoder-layer shape: 1024 groups of 4 target series plus their known-future covariate
    (5 rows each), 2048-step contexts fully observed (128 patches) + [REG] + 4 future patches = 133
    tokens; Chronos-2 120M-class layer (d_model 768, 12 x 64, d_ff 3072), weights N(0, 0.02), norm
    weights 1, activations x ~ N(0, 1)."""
    import torch

    from .chronos2 import layer_workspace_bytes

    rows, n, inner = groups * per_group, nc + 1 + h, heads * dh
    x = torch.empty(rows * n, d, dtype=torch.float32, device=device)
    fill_normal(x, rng.stream_seed(seed, 10), 0.0, 1.0)
    shapes = {"time_qkv": (3 * inner, d), "time_o": (d, inner), "group_qkv": (3 * inner, d), "group_o": (d, inner),
              "wi": (dff, d), "wo": (d, dff)}
    weights = {}
    for i, (name, shape) in enumerate(shapes.items()):
        t = torch.empty(shape, dtype=torch.float32, device=device)
        fill_normal(t, rng.stream_seed(seed, 11 + i), 0.0, 0.02)
        weights[name] = t
    for name in ("time_norm", "group_norm", "mlp_norm"):
        weights[name] = torch.ones(d, dtype=torch.float32, device=device)
    live = torch.ones(rows * n, dtype=torch.int32, device=device)
    starts = (np.arange(rows) // per_group * per_group).astype(np.int32)
    gs = torch.from_numpy(starts).to(device)
    ge = torch.from_numpy(starts + per_group).to(device)
    table = torch.from_numpy(rope_table(n, dh)).to(device)
    ws = torch.empty(layer_workspace_bytes(rows, n, d, inner, dff) // 4 + 64, dtype=torch.float32, device=device)
    return LayerCase(rows, n, heads, dh, d, dff, groups, x, weights, live, table, gs, ge, ws)


@dataclass
class TsTimeCase:
    rows: int
    n: int
    heads: int
    dh: int
    d: int
    qkv: object  # torch bf16 [rows*n, 3*d]
    gate: object  # torch bf16 [rows*n, d]
    key_valid: object  # torch int32 [rows*n]
    known: object  # torch int32 [rows]
    pos: object  # torch int32 [rows*n]: table rows (position + n)
    table: object  # torch float32 [2n, dh]
    starts: np.ndarray

    def mask_aware_flops(self) -> float:
        """4*dh per (row, head, query, allowed key): every valid key (k >= start, known rows read
        both directions) plus the query itself where it is not a valid key."""
        per_row = [(self.n - s) * self.n + s for s in self.starts]
        return 4.0 * self.dh * self.heads * float(sum(per_row))


def ts_time_config3(rows: int = 64, n: int = 1024, heads: int = 12, dh: int = 64, d: int = 768, rope_dim: int = 32,
                    max_start: int = 256, seed: int = 0, device: str = "cuda") -> TsTimeCase:
    """Config 3's time-attention sublayer: Timestral 123M-class (d_model 768, 12 x 64,
    rope_partial_factor 0.5), 64 series x 1024 patch tokens, x ~ N(0, 1), projections N(0, 0.02),
    q|k|v and the gate projection in bf16; bidirectional (every row a known covariate, so each
    query reads every valid key) with left padding U{0..256} masked (attend_missing_patches: keys
    from the first observed patch on are valid); positions count from the first observed patch."""
    import torch

    from .timestral import rope_table as ts_rope_table

    x = torch.empty(rows * n, d, dtype=torch.float32, device=device)
    w = torch.empty(4 * d, d, dtype=torch.float32, device=device)
    fill_normal(x, rng.stream_seed(seed, 20), 0.0, 1.0)
    fill_normal(w, rng.stream_seed(seed, 21), 0.0, 0.02)
    proj = (x @ w.t()).to(torch.bfloat16)
    del x, w
    qkv = proj[:, : 3 * d].contiguous()
    gate = proj[:, 3 * d:].contiguous()
    del proj
    starts = rng.randint(rng.stream_seed(seed, 22), rows, 0, max_start)
    t = np.arange(n)[None, :]
    key_valid = (t >= starts[:, None]).astype(np.int32)
    pos = (t - starts[:, None] + n).astype(np.int32)  # table row = position + enc
    known = np.ones(rows, np.int32)
    table = torch.from_numpy(ts_rope_table(n, n, dh, rope_dim)).to(device)
    return TsTimeCase(rows, n, heads, dh, d, qkv, gate, torch.from_numpy(key_valid.reshape(-1)).to(device),
                      torch.from_numpy(known).to(device), torch.from_numpy(pos.reshape(-1)).to(device), table, starts)


def c2_forecast_config4(groups: int = 1024, per_group: int = 4, t: int = 2048, horizon: int = 64, seed: int = 0):
    """Config 4's forecast inputs (host arrays): each group holds `per_group` target series of `t`
    steps (config 0's generator: sines of periods 24 and 168 with amplitudes U(0.5, 2), a linear
    trend of slope U(-0.01, 0.01), N(0, 0.1) noise) and one known-future covariate row (N(0, 1) past
    and `horizon` future steps). Returns (context [rows, t], group [rows], future [rows, horizon],
    targets: the boolean mask of target rows)."""
    r = np.random.default_rng(seed)
    rows = groups * (per_group + 1)
    steps = np.arange(t, dtype=np.float64)
    ctx = np.empty((rows, t), np.float32)
    fut = np.full((rows, horizon), np.nan, np.float32)
    targets = np.ones(rows, bool)
    for g in range(groups):
        base = g * (per_group + 1)
        for s in range(per_group):
            a1, a2 = r.uniform(0.5, 2.0, 2)
            slope = r.uniform(-0.01, 0.01)
            ctx[base + s] = (a1 * np.sin(2 * np.pi * steps / 24) + a2 * np.sin(2 * np.pi * steps / 168) + slope * steps
                             + r.normal(0, 0.1, t)).astype(np.float32)
        cov = base + per_group
        ctx[cov] = r.standard_normal(t).astype(np.float32)
        fut[cov] = r.standard_normal(horizon).astype(np.float32)
        targets[cov] = False
    group = (np.arange(rows) // (per_group + 1)).astype(np.int32)
    return ctx, group, fut, targets


def c2_portable_weights(c, seed: int = 0, std: float = 0.02) -> dict:
    """Chronos-2 random-init weights from the portable RNG, so every language of a build draws the
    same values: `shared` and every linear weight N(0, std) (tensor k of the binding order on stream
    seed * 1000003 + 100 + k), RMSNorm weights 1, biases 0 (config 0's recorded choice). The layout is
    HipChronos2Model's (q|k|v fused per attention sublayer)."""
    from .checkpoint import _chronos2_names

    w: dict = {"layers": [dict() for _ in range(c.num_layers)]}
    for k, (name, shape, key) in enumerate(_chronos2_names(c)):
        if name.endswith(".bias"):
            arr = np.zeros(shape, np.float32)
        elif "layer_norm" in name:
            arr = np.ones(shape, np.float32)
        else:
            count = int(np.prod(shape))
            arr = rng.normal(rng.stream_seed(seed, 100 + k), count, std).reshape(shape)
        if isinstance(key, tuple):
            w["layers"][key[0]][key[1]] = arr
        else:
            w[key] = arr
    for lw in w["layers"]:
        for kind in ("time", "group"):
            lw[f"{kind}_qkv"] = np.concatenate([lw.pop(f"{kind}_q"), lw.pop(f"{kind}_k"), lw.pop(f"{kind}_v")])
    return w


def c2_config0_series(rows: int = 4, t: int = 512, seed: int = 0) -> np.ndarray:
    """Config 0's inputs from the portable RNG: per series A1 sin(2 pi t / 24) + A2 sin(2 pi t / 168) +
    s t + eps with A1, A2 ~ U(0.5, 2), s ~ U(-0.01, 0.01), eps ~ N(0, 0.1), in double, rounded to
    float. Returns float32 [rows, t]."""
    amp = rng.uniform_range(rng.stream_seed(seed, 40), 2 * rows, 0.5, 2.0).reshape(rows, 2)
    slope = rng.uniform_range(rng.stream_seed(seed, 41), rows, -0.01, 0.01)
    noise = rng.normal(rng.stream_seed(seed, 42), rows * t, 0.1).reshape(rows, t).astype(np.float64)
    steps = np.arange(t, dtype=np.float64)
    x = (amp[:, :1] * np.sin(2 * np.pi * steps / 24) + amp[:, 1:] * np.sin(2 * np.pi * steps / 168)
         + slope[:, None] * steps + noise)
    return x.astype(np.float32)
