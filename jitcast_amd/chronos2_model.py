"""The Chronos-2 forward on libjitcast_hip: the host ends of Chronos2Model.forward and an engine that
runs the encoder on the GPU, the way the reference's Chronos2Forward.Plan does.

  Chronos2Config          the fields of Chronos2Config (J/chronos2/Chronos2Config.java:48-63) this
                          forward needs, with Chronos-2's published defaults
  random_weights          seeded random-init weights in Chronos2Weights' shapes
                          (J/chronos2/Chronos2Weights.java:77-100)
  layout                  ModelLayout.of (J/chronos2/ModelLayout.java:70-116): the cut, NaN-padded
                          context, the future covariates, the live mask
  prep, finish            ModelPrep.of / finish (J/chronos2/ModelPrep.java:38-151): instance norm,
                          patch tokens, inverse norm
  HipChronos2Model        the device forward: input patch embedding (jc_c2_residual), token
                          assembly (jc_c2_assemble), the encoder layers (jc_c2_layer), final norm
                          (jc_rms_norm), future gather (jc_c2_gather_future), output patch embedding
                          (jc_c2_residual); the order of Chronos2Forward.Plan's task graph
                          (J/chronos2/tornado/Chronos2Forward.java:250-292)

The host ends are numpy restatements with the reference's float32/double rounding; everything
between them runs on the GPU through the C ABI.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import _lib, chronos2, runtime
from . import options as opts
from . import plans as plans_mod

QUANTILES_21 = (0.01, 0.05, 0.1, 0.15, 0.2, 0.25, 0.3, 0.35, 0.4, 0.45, 0.5, 0.55, 0.6, 0.65, 0.7, 0.75, 0.8, 0.85,
                0.9, 0.95, 0.99)


@dataclass(frozen=True)
class Chronos2Config:
    d_model: int = 768
    d_kv: int = 64
    d_ff: int = 3072
    num_layers: int = 12
    num_heads: int = 12
    layer_norm_eps: float = float(np.float32(1e-6))  # Chronos2Config keeps it as a float
    rope_theta: float = 10000.0
    context_length: int = 8192
    patch_size: int = 16
    max_output_patches: int = 64
    quantiles: tuple = QUANTILES_21
    use_reg_token: bool = True
    use_arcsinh: bool = True
    time_encoding_scale: int = 8192

    @property
    def inner(self) -> int:
        return self.num_heads * self.d_kv

    @property
    def num_quantiles(self) -> int:
        return len(self.quantiles)

    @property
    def vocab_size(self) -> int:
        return 2 if self.use_reg_token else 1

    def quantile_levels(self) -> np.ndarray:
        """The levels as forecasts report them: each double rounded to float (Chronos2Config.quantileLevels)."""
        return np.asarray(self.quantiles, np.float64).astype(np.float32)

    def prediction_length(self) -> int:
        """The steps one forward pass forecasts before the long-horizon unrolling."""
        return self.max_output_patches * self.patch_size

    @staticmethod
    def from_json(text: str) -> "Chronos2Config":
        """Chronos2Config.fromJson (J/chronos2/Chronos2Config.java:118-166): a config.json document with
        only the known keys (unknown ones fail), a Chronos2Model with the ReLU feed-forward layer,
        float32 weights, equal input/output patch sizes and stride; the missing values take the
        reference's defaults. ValueError on anything else."""
        from .checkpoint import parse_config

        return parse_config(text)

    @staticmethod
    def load(path) -> "Chronos2Config":
        """Chronos2Config.load: from_json of the file at path."""
        from pathlib import Path

        return Chronos2Config.from_json(Path(path).read_text(encoding="utf-8"))


def random_weights(c: Chronos2Config, seed: int = 0, std: float = 0.02) -> dict:
    """Seeded N(0, std) matrices and biases, norm weights 1, in Chronos2Weights' shapes: `shared`
    [vocab, d] (row 1 is [REG]), the input and output residual blocks (`in_*`, `out_*`: hidden,
    output and residual linears with biases), `layers` (dicts keyed like jc_c2_layer_weights, no
    biases) and `final_norm`."""
    r = np.random.default_rng(seed)
    d, ff, p, inner = c.d_model, c.d_ff, c.patch_size, c.inner

    def m(o, i):
        return (std * r.standard_normal((o, i))).astype(np.float32)

    def b(o):
        return (std * r.standard_normal(o)).astype(np.float32)

    w = {"shared": m(c.vocab_size, d), "final_norm": np.ones(d, np.float32)}
    for pre, din, dout in (("in", 3 * p, d), ("out", d, c.num_quantiles * p)):
        w[f"{pre}_hidden_w"], w[f"{pre}_hidden_b"] = m(ff, din), b(ff)
        w[f"{pre}_output_w"], w[f"{pre}_output_b"] = m(dout, ff), b(dout)
        w[f"{pre}_residual_w"], w[f"{pre}_residual_b"] = m(dout, din), b(dout)
    w["layers"] = [{
        "time_norm": np.ones(d, np.float32), "time_qkv": m(3 * inner, d), "time_o": m(d, inner),
        "group_norm": np.ones(d, np.float32), "group_qkv": m(3 * inner, d), "group_o": m(d, inner),
        "mlp_norm": np.ones(d, np.float32), "wi": m(ff, d), "wo": m(d, ff),
    } for _ in range(c.num_layers)]
    return w


@dataclass
class Layout:
    rows: int
    nc: int
    nreg: int
    h: int
    window: np.ndarray  # [rows, nc*P] float32, NaN where missing
    future: np.ndarray  # [rows, h*P] float32, NaN where unknown
    live: np.ndarray  # [rows, n] int32
    group: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))

    @property
    def n(self) -> int:
        return self.nc + self.nreg + self.h

    @property
    def future_start(self) -> int:
        return self.nc + self.nreg


def layout(c: Chronos2Config, context, group, future_covariates=None, h: int = 1) -> Layout:
    """ModelLayout.of: the most recent context_length steps, NaN-padded on the left to whole
    patches; the future covariates (NaN where unknown); every token live except a context patch
    with no observed value. Errors are ModelLayout's IllegalArgumentExceptions."""
    if h < 1:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"output patches must be >= 1, got {h}")
    ctx = np.asarray(context, np.float32)
    rows, t = ctx.shape
    group = np.asarray(group, np.int32)
    if group.shape != (rows,):
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "group ids must have one entry per row")
    ps = c.patch_size
    kept = min(t, c.context_length)
    padded = (kept + ps - 1) // ps * ps
    window = np.full((rows, padded), np.nan, np.float32)
    window[:, padded - kept:] = ctx[:, t - kept:]
    fut = np.full((rows, h * ps), np.nan, np.float32)
    if future_covariates is not None:
        fc = np.asarray(future_covariates, np.float32)
        if fc.ndim != 2 or fc.shape[0] != rows or fc.shape[1] > h * ps:
            raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"{h} output patches cannot hold {fc.shape[-1]} future steps")
        fut[:, : fc.shape[1]] = fc
    nc = padded // ps
    nreg = 1 if c.use_reg_token else 0
    live = chronos2.live_mask(window, nc, ps, nreg, h)
    return Layout(rows, nc, nreg, h, window, fut, live, group)


def _instance_norm(window: np.ndarray):
    """InstanceNorm per row: the mean and population std of the observed values in double, rounded
    to float; a zero std floored at 1e-5; (0, 1) for a row with none."""
    obs = ~np.isnan(window)
    cnt = obs.sum(axis=1)
    x64 = np.where(obs, window, 0).astype(np.float64)
    loc = np.where(cnt > 0, (x64.sum(axis=1) / np.maximum(cnt, 1)), 0.0).astype(np.float32)
    dev = np.where(obs, (window - loc[:, None]).astype(np.float32), np.float32(0)).astype(np.float64)
    scale = np.sqrt((dev * dev).sum(axis=1) / np.maximum(cnt, 1)).astype(np.float32)
    scale = np.where(cnt > 0, np.where(scale == 0, np.float32(1e-5), scale), np.float32(1)).astype(np.float32)
    return loc, scale


def _scaled(x: np.ndarray, loc: np.ndarray, scale: np.ndarray, arcsinh: bool) -> np.ndarray:
    v = ((x - loc) / scale).astype(np.float32)
    if arcsinh:
        a = np.abs(v.astype(np.float64))
        r = np.log(a + np.sqrt(a * a + 1.0))
        v = np.where(v < 0, -r, r).astype(np.float32)
    return v


def prep(c: Chronos2Config, lay: Layout):
    """ModelPrep.of: tokens [rows*(nc+h), 3P] (time encoding, scaled value or 0, observed mask) of
    each row's context patches then its future patches, and loc, scale [rows]."""
    ps, nc, h, rows = c.patch_size, lay.nc, lay.h, lay.rows
    loc, scale = _instance_norm(lay.window)
    ts = np.float32(c.time_encoding_scale)
    tok = np.zeros((rows, nc + h, 3 * ps), np.float32)
    t_ctx = np.arange(nc * ps)
    tok[:, :nc, :ps] = ((t_ctx - nc * ps).astype(np.float32) / ts).reshape(nc, ps)
    obs = ~np.isnan(lay.window)
    val = np.where(obs, _scaled(np.nan_to_num(lay.window), loc[:, None], scale[:, None], c.use_arcsinh), np.float32(0))
    tok[:, :nc, ps:2 * ps] = val.reshape(rows, nc, ps)
    tok[:, :nc, 2 * ps:] = obs.astype(np.float32).reshape(rows, nc, ps)
    t_fut = np.arange(h * ps)
    tok[:, nc:, :ps] = (t_fut.astype(np.float32) / ts).reshape(h, ps)
    fobs = ~np.isnan(lay.future)
    fval = np.where(fobs, _scaled(np.nan_to_num(lay.future), loc[:, None], scale[:, None], c.use_arcsinh), np.float32(0))
    tok[:, nc:, ps:2 * ps] = fval.reshape(rows, h, ps)
    tok[:, nc:, 2 * ps:] = fobs.astype(np.float32).reshape(rows, h, ps)
    return tok.reshape(rows * (nc + h), 3 * ps), loc, scale


def finish(c: Chronos2Config, lay: Layout, raw: np.ndarray, loc: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """ModelPrep.finish: raw [rows*h, Q*P] (quantiles level-major per token) -> [rows, Q, h*P] as
    sinh(x)*scale + loc (without sinh when the model does not use arcsinh)."""
    rows, h, q, ps = lay.rows, lay.h, c.num_quantiles, c.patch_size
    v = raw.reshape(rows, h, q, ps).astype(np.float32)
    if c.use_arcsinh:
        v = np.sinh(v.astype(np.float64)).astype(np.float32)
    out = (v * scale[:, None, None, None] + loc[:, None, None, None]).astype(np.float32)
    return out.transpose(0, 2, 1, 3).reshape(rows, q, h * ps)


class HipChronos2Model:
    """The Chronos-2 forward on one GPU: weights uploaded once; per call the host prep, one upload,
    the device forward, one download and the host finish. dtype "f32" runs every layer in fp32;
    "bf16"/"fp16" runs the encoder layers' GEMMs and time attention in that type with fp32
    accumulation (the reference's FP16 GEMM mode), the embeddings and head in fp32; "f16x3" runs the
    layers' GEMMs on three-term fp16 splits of their operands (fp32 accumulation and outputs, about
    fp32's accuracy) and everything else as "f32"."""

    def __init__(self, c: Chronos2Config, weights: dict, dtype: str = "f32", device: int = 0, max_plans: int = 0,
                 plan_bytes: int | None = None):
        """max_plans > 0 runs the device forward as captured plans, one hipGraph per
        Shape(rows, contextPatches, outputPatches) (Chronos2Forward.Shape, Chronos2Forward.java:106),
        kept in a PlanCache of at most max_plans plans within plan_bytes of plan buffers
        (Chronos2Forward.java:108-113; default: no byte limit). The weights are uploaded once and
        shared by every plan, so a plan's footprint is its shape's buffers only."""
        import torch

        self.c, self.dtype = c, dtype
        self.code = {"f32": _lib.JC_F32, "bf16": _lib.JC_BF16, "fp16": _lib.JC_F16, "f16x3": _lib.JC_F16X3}[dtype]
        self.dev = torch.device("cuda", device)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)  # noqa: E731
        self.w = {k: t(v) for k, v in weights.items() if k != "layers"}
        self.reg = self.w["shared"][1].contiguous() if c.use_reg_token else None
        self.layers = []
        for lw in weights["layers"]:
            d = {k: t(v) for k, v in lw.items()}
            if self.code == _lib.JC_F16X3:
                for k in ("time_qkv", "time_o", "group_qkv", "group_o", "wi", "wo"):
                    src = d[k].contiguous()
                    x3 = torch.empty(src.shape[0], 3 * src.shape[1], dtype=torch.float16, device=self.dev)
                    chronos2.split_f16x3(src, x3, weights=True)
                    d[k] = x3
            elif self.code != _lib.JC_F32:
                tdt = {_lib.JC_BF16: torch.bfloat16, _lib.JC_F16: torch.float16}[self.code]
                for k in ("time_qkv", "time_o", "group_qkv", "group_o", "wi", "wo"):
                    lp = torch.empty(d[k].shape, dtype=tdt, device=self.dev)
                    chronos2.to_lp(d[k], lp)
                    d[k] = lp
            self.layers.append(d)
        self._bufs = {}
        # -Dchronos2.hip.profile: per-kernel times of each eager forward, the time of each plan replay
        self.profile = opts.boolean("chronos2.hip.profile", False)
        self.plans = None
        if max_plans > 0:
            self.plans = plans_mod.PlanCache(max_plans, plan_bytes if plan_bytes else 1 << 62)
            self._stream = torch.cuda.Stream(self.dev)  # default priority; plans capture and replay on it

    def _alloc(self, rows: int, nc: int, h: int, inputs: bool = False) -> dict:
        """One shape's device buffers (Chronos2Forward.Plan's, Chronos2Forward.java:206-236); with
        inputs, also the forward's inputs (tokens, live, group bounds) that a plan replays from."""
        import torch

        c = self.c
        nreg = 1 if c.use_reg_token else 0
        n = nc + nreg + h
        ne, d, ff = nc + h, c.d_model, c.d_ff
        f = lambda *s: torch.empty(*s, dtype=torch.float32, device=self.dev)  # noqa: E731
        ws = chronos2.layer_workspace_bytes(rows, n, d, c.inner, ff, self.code)
        b = {
            "emb": f(rows * ne, d), "scratch": f(rows * max(ne, h), ff), "x": f(rows * n, d),
            "y": f(rows * n, d), "dec": f(rows * h, d), "raw": f(rows * h, c.num_quantiles * c.patch_size),
            "ws": f(ws // 4 + 64), "table": torch.from_numpy(chronos2.rope_table(n, c.d_kv, c.rope_theta)).to(self.dev),
        }
        if inputs:
            i32 = lambda m: torch.empty(m, dtype=torch.int32, device=self.dev)  # noqa: E731
            b.update({"tok": f(rows * ne, 3 * c.patch_size), "live": i32(rows * n), "gs": i32(rows), "ge": i32(rows)})
        return b

    def _buffers(self, rows: int, nc: int, h: int):
        key = (rows, nc, h)
        if key not in self._bufs:
            self._bufs.clear()  # the eager forward keeps one shape's buffers
            self._bufs[key] = self._alloc(rows, nc, h)
        return self._bufs[key]

    def forward_raw(self, tokens, live, group_start, group_end, rows: int, nc: int, h: int, bufs: dict | None = None,
                    sink=None):
        """The device forward from prepared tokens (torch [rows*(nc+h), 3P] on the GPU) to the raw
        output patch embedding [rows*h, Q*P] on the GPU; rows grouped contiguously. bufs: a plan's
        buffers (default: the eager forward's). sink(name, x), when given, sees the encoder's x after
        each layer ("layer0", ...), as the reference's StageSink (CpuChronos2.java:160)."""
        label = f"chronos2.hip.profile forward rows={rows} n={nc + (1 if self.c.use_reg_token else 0) + h}"
        with runtime.kernel_profile(self.dev.index or 0, label, self.profile):
            return self._forward_raw(tokens, live, group_start, group_end, rows, nc, h, bufs, sink)

    def _forward_raw(self, tokens, live, group_start, group_end, rows: int, nc: int, h: int, bufs, sink):
        c = self.c
        nreg = 1 if c.use_reg_token else 0
        n, ne, d, ff = nc + nreg + h, nc + h, c.d_model, c.d_ff
        b = bufs if bufs is not None else self._buffers(rows, nc, h)
        w = self.w
        ctx = chronos2.context(self.dev.index or 0)
        p = chronos2._ptr
        _lib.call("jc_c2_residual", ctx.handle, p(tokens), rows * ne, 3 * c.patch_size, p(w["in_hidden_w"]),
                  p(w["in_hidden_b"]), p(w["in_output_w"]), p(w["in_output_b"]), p(w["in_residual_w"]),
                  p(w["in_residual_b"]), ff, d, p(b["scratch"]), p(b["emb"]))
        _lib.call("jc_c2_assemble", ctx.handle, p(b["emb"]), p(self.reg), p(b["x"]), rows, nc, nreg, n, d)
        for li, lw in enumerate(self.layers):
            chronos2.layer(b["x"], lw, live, b["table"], group_start, group_end, b["ws"], rows, n, d, c.num_heads,
                           c.d_kv, ff, c.layer_norm_eps, self.code)
            if sink is not None:
                sink(f"layer{li}", b["x"])
        chronos2.rms_norm(b["x"], w["final_norm"], b["y"], c.layer_norm_eps)
        _lib.call("jc_c2_gather_future", ctx.handle, p(b["y"]), p(b["dec"]), rows, nc + nreg, n, h, d)
        _lib.call("jc_c2_residual", ctx.handle, p(b["dec"]), rows * h, d, p(w["out_hidden_w"]), p(w["out_hidden_b"]),
                  p(w["out_output_w"]), p(w["out_output_b"]), p(w["out_residual_w"]), p(w["out_residual_b"]), ff,
                  c.num_quantiles * c.patch_size, p(b["scratch"]), p(b["raw"]))
        return b["raw"]

    def forecast(self, context, group, future_covariates=None, h: int = 1) -> np.ndarray:
        """Quantile forecasts [rows, Q, h*P] for the input rows (group ids per row; rows of a group
        need not be adjacent: they are ordered as Chronos2Forward.groupOrder orders them and the
        results are put back in input order). The host ends run on the device too (jc_c2_prep,
        jc_c2_finish): only the raw rows go up and the finished quantiles come down."""
        import torch

        c = self.c
        ctx, group, fut = _check_inputs(c, context, group, future_covariates, h)
        rows = ctx.shape[0]
        order = chronos2.group_order(group)
        gs, ge = chronos2.group_bounds(group[order] if order is not None else group)
        dev = self.dev
        up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        ord_t = up(order) if order is not None else None
        nreg = 1 if c.use_reg_token else 0
        if self.plans is not None:
            with torch.cuda.stream(self._stream):
                return self._forecast_planned(ctx, fut, order, gs, ge, rows, h)
        tok, loc, scale, live, nc = chronos2.prep(up(ctx), up(fut) if fut is not None else None, ord_t, rows,
                                                  c.context_length, c.patch_size, h, nreg, c.time_encoding_scale,
                                                  c.use_arcsinh)
        raw = self.forward_raw(tok, live, up(gs), up(ge), rows, nc, h)
        out = torch.empty(rows, c.num_quantiles, h * c.patch_size, dtype=torch.float32, device=dev)
        chronos2.finish(raw, loc, scale, ord_t, rows, h, c.num_quantiles, c.patch_size, c.use_arcsinh, out)
        return out.cpu().numpy()

    def _forecast_planned(self, ctx, fut, order, gs, ge, rows: int, h: int) -> np.ndarray:
        """forecast through the plan of its shape (Chronos2Forward.forward's plans.run): the
        uploads and jc_c2_prep, then the plan's forward replayed on its own buffers (captured on the
        shape's first use), then jc_c2_finish. Runs on the model's stream."""
        import torch

        c = self.c
        dev = self.dev
        up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        ord_t = up(order) if order is not None else None
        nreg = 1 if c.use_reg_token else 0
        tok, loc, scale, live, nc = chronos2.prep(up(ctx), up(fut) if fut is not None else None, ord_t, rows,
                                                  c.context_length, c.patch_size, h, nreg, c.time_encoding_scale,
                                                  c.use_arcsinh)
        shape = (rows, nc, h)

        def use(plan: ShapePlan):
            b = plan.bufs
            b["tok"].copy_(tok)
            b["live"].copy_(live)
            b["gs"].copy_(up(gs))
            b["ge"].copy_(up(ge))
            runtime.timed_replay(f"chronos2.hip.profile rows={rows} nc={nc} h={h}", self.profile, plan.graph.launch)
            out = torch.empty(rows, c.num_quantiles, h * c.patch_size, dtype=torch.float32, device=dev)
            chronos2.finish(b["raw"], loc, scale, ord_t, rows, h, c.num_quantiles, c.patch_size, c.use_arcsinh, out)
            return out.cpu().numpy()

        return self.plans.run(shape, self._capture, use)

    def _capture(self, shape) -> "ShapePlan":
        """Chronos2Forward.Plan's constructor: the shape's buffers, then the device forward captured
        into one hipGraph on the model's stream (nothing allocates while it captures)."""
        import torch

        rows, nc, h = shape
        b = self._alloc(rows, nc, h, inputs=True)
        with torch.cuda.stream(self._stream):
            with plans_mod.capture((rows << 40) | (nc << 20) | h, self.dev.index or 0) as box:
                self.forward_raw(b["tok"], b["live"], b["gs"], b["ge"], rows, nc, h, bufs=b)
        return ShapePlan(box[0], b)

    def close(self) -> None:
        """Closes every cached plan (Chronos2Forward.close)."""
        if self.plans is not None:
            self.plans.close()


class ShapePlan:
    """One shape's captured forward and the buffers it replays on (PlanCache.Plan): its footprint
    is those buffers plus what the graph adopted; the weights are not counted, being shared."""

    def __init__(self, graph, bufs: dict):
        self.graph, self.bufs = graph, bufs

    def device_bytes(self) -> int:
        return self.graph.device_bytes() + sum(t.numel() * t.element_size() for t in self.bufs.values())

    def close(self) -> None:
        self.graph.close()
        self.bufs = {}


def _check_inputs(c: Chronos2Config, context, group, future_covariates, h: int):
    """The argument checks of ModelLayout.of (J/chronos2/ModelLayout.java:70-116): at least one
    output patch, one group id per row, no more known future steps than h patches hold."""
    if h < 1:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"output patches must be >= 1, got {h}")
    ctx = np.asarray(context, np.float32)
    if ctx.ndim != 2:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "context must be [rows, steps]")
    group = np.ascontiguousarray(np.asarray(group, np.int32))
    if group.shape != (ctx.shape[0],):
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "group ids must have one entry per row")
    fut = None
    if future_covariates is not None:
        fut = np.asarray(future_covariates, np.float32)
        if fut.ndim != 2 or fut.shape[0] != ctx.shape[0] or fut.shape[1] > h * c.patch_size:
            raise _lib.JitcastArgumentError(_lib.JC_EINVAL,
                                            f"{h} output patches cannot hold {fut.shape[-1]} future steps")
    return ctx, group, fut
