"""The Timestral block forward on libjitcast_hip: the device half of TimestralModel.predict_block,
run the way the reference's TimestralForward.Plan queues it (J/timestral/tornado/
TimestralForward.java:327-382).

  TimestralConfig     the fields of TimestralConfig (J/timestral/TimestralConfig.java:53-71) this
                      forward needs; the defaults are the 123M-class shape of the benchmark configs
  random_weights      seeded random-init weights in the engine's layouts (TimestralWeights.qkv and
                      mlpUp's rearranged copies, J/timestral/TimestralWeights.java:150-186)
  HipTimestralModel   the device forward from patch tokens to the head's raw outputs:
                      patch embedding (jc_ts_residual), token assembly (jc_ts_assemble), per layer
                      each attention sublayer (jc_rms_norm, jc_linear q|k|v and gate projection,
                      jc_ts_time_attention or jc_ts_variate_attention with the gate fused,
                      jc_linear output projection accumulated) and the SwiGLU MLP (jc_linear,
                      jc_swiglu, jc_linear accumulated), the output norm, the decoder tokens
                      (jc_ts_gather_decoder) and the head (jc_ts_residual)

  block_window        BlockLayout.of's window (J/timestral/BlockLayout.java:77-148) on the host
  block_prep, quantile_map, block_finish
                      numpy restatements of BlockPrep.of (BlockPrep.java:40-75; Scaler.java's causal
                      patch loc/scale, instance norm, affine), Quantiles.apply (Quantiles.java:52-77)
                      and BlockPrep.finish (BlockPrep.java:77-101; Scaler.invert, clampNonFinite),
                      with the reference's float/double rounding, for callers that hold the block on
                      the host; predict_block runs the device versions (jc_ts_prep, jc_ts_finish)
  HipTimestralModel.predict_block
                      the window and BlockLayout on the host, then BlockPrep, the forward and finish
                      on the device
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib, chronos2, chronos2_model, runtime, timestral
from . import options as opts
from . import plans as plans_mod

QUANTILES_9 = (0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9)


@dataclass(frozen=True)
class TimestralConfig:
    patch_size: int = 16
    d_model: int = 768
    num_heads: int = 12
    mlp_hidden_dim: int = 3072
    # per layer, per attention sublayer: True = time attention, False = variate attention
    layers: tuple = ((True, False),) * 12
    quantiles: tuple = QUANTILES_9
    rope_theta: float = 10000.0
    rope_partial_factor: float = 0.5
    norm_eps: float = 1e-6
    time_attn_gate: bool = True
    variate_attn_gate: bool = True
    minimum_scale: float = 1e-6
    use_asinh: bool = True
    quantile_width_factor: float = 2.0
    covariate_enabled: bool = True
    attend_missing: bool = True
    block_size: int = 64
    context_length: int = 16384  # steps the pipeline keeps by default (Options.maxContext)

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    @property
    def rope_dim(self) -> int:
        return int(self.head_dim * self.rope_partial_factor)

    @property
    def num_quantiles(self) -> int:
        return len(self.quantiles)

    @property
    def median_index(self) -> int:
        return self.quantiles.index(0.5)

    def supports_known_covariates(self) -> bool:
        """TimestralConfig.supportsKnownCovariates (TimestralConfig.java:129-148): covariates on, and a time
        attention followed later by both a time and a variate attention."""
        if not self.covariate_enabled:
            return False
        ops = [bool(t) for axes in self.layers for t in axes]
        return any(ops[i] and True in ops[i + 1:] and False in ops[i + 1:] for i in range(len(ops)))


def random_weights(c: TimestralConfig, seed: int = 0, std: float = 0.02) -> dict:
    """Seeded N(0, std) matrices, norm scales 1 + N(0, std), in the engine's layouts: the patch
    embedding (`embed_*`: hidden [4d, 2P], output [d, 4d], residual [d, 2P], with biases), the
    forecast `query` [d], `layers` (each a dict of `attentions`, a list of {time, norm, qkv [3d, d]
    heads-major q|k|v, gate [d, d] or None, wo [d, d]}, and the MLP's `mlp_norm`, `up` [2f, d] with
    the SiLU half first, `down` [d, f]), `out_norm` and the head (`head_*`: hidden [4d, d], output
    [P*Q, 4d], residual [P*Q, d], no biases). TimestralWeights binds the same shapes
    (TimestralWeights.java:92-117)."""
    r = np.random.default_rng(seed)
    d, p, f = c.d_model, c.patch_size, c.mlp_hidden_dim

    def m(o, i):
        return (std * r.standard_normal((o, i))).astype(np.float32)

    def v(o, base=0.0):
        return (base + std * r.standard_normal(o)).astype(np.float32)

    w = {"query": v(d), "out_norm": v(d, 1.0)}
    for pre, din, hid, dout, bias in (("embed", 2 * p, 4 * d, d, True), ("head", d, 4 * d, p * c.num_quantiles, False)):
        w[f"{pre}_hidden_w"], w[f"{pre}_output_w"], w[f"{pre}_residual_w"] = m(hid, din), m(dout, hid), m(dout, din)
        if bias:
            w[f"{pre}_hidden_b"], w[f"{pre}_output_b"], w[f"{pre}_residual_b"] = v(hid), v(dout), v(dout)
    w["layers"] = []
    for axes in c.layers:
        attns = []
        for time in axes:
            gated = c.time_attn_gate if time else c.variate_attn_gate
            attns.append({"time": bool(time), "norm": v(d, 1.0), "qkv": m(3 * d, d), "gate": m(d, d) if gated else None,
                          "wo": m(d, d)})
        w["layers"].append({"attentions": attns, "mlp_norm": v(d, 1.0), "up": m(2 * f, d), "down": m(d, f)})
    return w


class HipTimestralModel:
    """The Timestral block forward on one GPU: weights uploaded once, per-shape buffers kept for the
    last shape, one call per block. dtype "f32" is the reference's FP32-exact default; "bf16" /
    "fp16" mirror its FP16 GEMM mode (TimestralForward.java:467-499 with Kernels.gemmHalf): the
    attention sublayers' and the MLP's GEMMs take storage-type operands with fp32 accumulation, the
    time attention and SwiGLU run in the storage type, the variate attention reads fp32 q|k|v, the
    residual stream, norms' inputs, the embedding and the head stay fp32. "f16x3" (no reference
    counterpart) keeps every activation fp32 and runs each of those GEMMs on fp16 MFMA over
    three-term splits of its operands (weights split once at load, [hi | lo | hi]; the A operand
    split after its norm, attention or SwiGLU, [hi | hi | lo]): about fp32's accuracy."""

    def __init__(self, c: TimestralConfig, weights: dict, dtype: str = "f32", device: int = 0,
                 max_plans: int | None = None, plan_bytes: int | None = None, buckets: bool | None = None):
        """max_plans > 0 runs predict_block's device forward from captured plans, one hipGraph per
        Shape(rows, encoder, horizon, covariates) (TimestralForward.Shape, TimestralForward.java:135),
        kept in a PlanCache of at most max_plans within plan_bytes of plan buffers; the weights are
        uploaded once and shared by every plan. The defaults are the reference's: -Dtimestral.hip.plans
        (8) and -Dtimestral.hip.planBytes (the device's memory). buckets (default
        -Dtimestral.hip.buckets, true) pads each block to a shared shape first (bucketed,
        TimestralForward.java:81-99, 186-232)."""
        import torch

        self.c, self.dtype = c, dtype
        self.code = {"f32": _lib.JC_F32, "bf16": _lib.JC_BF16, "fp16": _lib.JC_F16, "f16x3": _lib.JC_F16X3}[dtype]
        self.tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16, "f16x3": torch.float16}[dtype]
        self.dev = torch.device("cuda", device)
        t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)  # noqa: E731

        def lp(a):  # a weight matrix in the storage type, converted once (Kernels.toHalf)
            if a is None or self.code == _lib.JC_F32:
                return t(a)
            src = t(a)
            if self.code == _lib.JC_F16X3:  # its three-term fp16 split [hi | lo | hi], [n, 3k]
                dst = torch.empty(src.shape[0], 3 * src.shape[1], dtype=torch.float16, device=self.dev)
                chronos2.split_f16x3(src, dst, weights=True)
                return dst
            dst = torch.empty(src.shape, dtype=self.tdt, device=self.dev)
            chronos2.to_lp(src, dst)
            return dst

        self.w = {k: t(v) for k, v in weights.items() if k != "layers"}
        self.layers = [{"attentions": [{"time": a["time"], "norm": t(a["norm"]), "qkv": lp(a["qkv"]), "gate": lp(a["gate"]),
                                        "wo": lp(a["wo"])} for a in lw["attentions"]],
                        "mlp_norm": t(lw["mlp_norm"]), "up": lp(lw["up"]), "down": lp(lw["down"])}
                       for lw in weights["layers"]]
        self._bufs = {}
        self.buckets = opts.boolean("timestral.hip.buckets", True) if buckets is None else bool(buckets)
        # -Dtimestral.hip.profile: per-kernel times of each eager forward, the time of each plan replay
        self.profile = opts.boolean("timestral.hip.profile", False)
        self.plans = None
        if max_plans is None:
            max_plans = opts.integer("timestral.hip.plans", 8, 0)
        if max_plans > 0:
            if plan_bytes is None:
                total = torch.cuda.get_device_properties(self.dev).total_memory
                plan_bytes = opts.bytes_("timestral.hip.planBytes", total, 1)
            self.plans = plans_mod.PlanCache(max_plans, plan_bytes)
            self._stream = torch.cuda.Stream(self.dev)  # default priority; plans capture and replay on it

    def _alloc(self, rows: int, enc: int, h: int, inputs: bool = False) -> dict:
        """One shape's device buffers; with inputs, also the per-call inputs a plan replays from
        (tokens, key validity, known rows, positions, group bounds, roles)."""
        import torch

        c = self.c
        n, d, f = enc + h, c.d_model, c.mlp_hidden_dim
        tokens = rows * n
        e = lambda *s: torch.empty(*s, dtype=torch.float32, device=self.dev)  # noqa: E731
        b = {
            "emb": e(rows * enc, d), "scratch": e(max(rows * enc, rows * h), 4 * d), "x": e(tokens, d),
            "hn": e(tokens, d), "big": e(tokens, max(3 * d, 2 * f)), "att": e(tokens, d), "gate": e(tokens, d),
            "act": e(tokens, f), "y": e(tokens, d), "dec": e(rows * h, d),
            "raw": e(rows * h, c.patch_size * c.num_quantiles),
            "table": torch.from_numpy(timestral.rope_table(enc, n, c.head_dim, c.rope_dim, c.rope_theta)).to(self.dev),
        }
        if self.code == _lib.JC_F16X3:  # the split of each GEMM's A operand, [tokens, 3k] fp16
            b["x3"] = torch.empty(tokens * 3 * max(d, f), dtype=torch.float16, device=self.dev)
        elif self.code != _lib.JC_F32:
            s = lambda *sh: torch.empty(*sh, dtype=self.tdt, device=self.dev)  # noqa: E731
            b.update({"hn_lp": s(tokens, d), "big_lp": s(tokens, max(3 * d, 2 * f)), "att_lp": s(tokens, d),
                      "gate_lp": s(tokens, d), "act_lp": s(tokens, f)})
        if inputs:
            i32 = lambda m: torch.zeros(m, dtype=torch.int32, device=self.dev)  # noqa: E731
            b.update({"tok": e(rows * enc, 2 * c.patch_size), "kv": i32(rows * enc), "known": i32(rows),
                      "pos": i32(rows * n), "gs": i32(rows), "ge": i32(rows), "role": i32(rows)})
        return b

    def _buffers(self, rows: int, enc: int, h: int):
        key = (rows, enc, h)
        if key not in self._bufs:
            self._bufs.clear()  # the eager forward keeps one shape's buffers
            self._bufs[key] = self._alloc(rows, enc, h)
        return self._bufs[key]

    def forward_raw(self, tokens, key_valid, known, pos, group_start, group_end, role, covariates: bool, rows: int,
                    enc: int, h: int, bufs: dict | None = None):
        """The device forward from the patch tokens (torch [rows*enc, 2P] on the GPU) to the head's
        raw outputs [rows*h, P*Q] on the GPU. key_valid [rows*enc], known [rows] (or None), pos
        [rows*(enc+h)] table rows from jc_ts_block_layout, group_start / group_end [rows] and role
        [rows] (or None) as int32 device tensors; rows of a series contiguous. bufs: a plan's buffers
        (default: the eager forward's)."""
        with runtime.kernel_profile(self.dev.index or 0, f"timestral.hip.profile forward rows={rows} n={enc + h}",
                                    self.profile):
            return self._forward_raw(tokens, key_valid, known, pos, group_start, group_end, role, covariates, rows,
                                     enc, h, bufs)

    def _forward_raw(self, tokens, key_valid, known, pos, group_start, group_end, role, covariates: bool, rows: int,
                     enc: int, h: int, bufs):
        c = self.c
        n, d = enc + h, c.d_model
        b = bufs if bufs is not None else self._buffers(rows, enc, h)
        w = self.w
        ctx = chronos2.context(self.dev.index or 0)
        p = chronos2._ptr
        _lib.call("jc_ts_residual", ctx.handle, p(tokens), rows * enc, 2 * c.patch_size, p(w["embed_hidden_w"]),
                  p(w.get("embed_hidden_b")), p(w["embed_output_w"]), p(w.get("embed_output_b")),
                  p(w["embed_residual_w"]), p(w.get("embed_residual_b")), 4 * d, d, p(b["scratch"]), p(b["emb"]))
        _lib.call("jc_ts_assemble", ctx.handle, p(b["emb"]), p(w["query"]), p(b["x"]), rows, enc, n, d)
        x = b["x"]
        self.encoder(x, key_valid, known, pos, group_start, group_end, role, covariates, rows, enc, h, bufs=b)
        chronos2.rms_norm(x, w["out_norm"], b["y"], c.norm_eps)
        _lib.call("jc_ts_gather_decoder", ctx.handle, p(b["y"]), p(b["dec"]), rows, enc, n, h, d)
        _lib.call("jc_ts_residual", ctx.handle, p(b["dec"]), rows * h, d, p(w["head_hidden_w"]), None,
                  p(w["head_output_w"]), None, p(w["head_residual_w"]), None, 4 * d, c.patch_size * c.num_quantiles,
                  p(b["scratch"]), p(b["raw"]))
        return b["raw"]

    def encoder(self, x, key_valid, known, pos, group_start, group_end, role, covariates: bool, rows: int, enc: int,
                h: int, mlp: bool = True, bufs: dict | None = None) -> None:
        """The encoder layers in place on x (torch fp32 [rows*(enc+h), d] on the GPU), in the order of
        TimestralForward.Plan's per-layer tasks (TimestralForward.java:335-382): each attention
        sublayer (RMSNorm, q|k|v and gate projections, time or variate attention with the gate fused,
        output projection accumulated into x), then the SwiGLU MLP unless mlp is False (the attention
        stack of the benchmark's config 3). Masks and positions as forward_raw takes them."""
        import torch

        c = self.c
        n, d, f, heads, dh = enc + h, c.d_model, c.mlp_hidden_dim, c.num_heads, c.head_dim
        ll = enc - h if covariates else enc
        tokens_n = rows * n
        if tuple(x.shape) != (tokens_n, d) or x.dtype != torch.float32 or not x.is_contiguous():
            raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"x must be fp32 [{tokens_n}, {d}]")
        b = bufs if bufs is not None else self._buffers(rows, enc, h)
        ctx = chronos2.context(self.dev.index or 0)
        p = chronos2._ptr
        x3 = self.code == _lib.JC_F16X3  # fp32 activations, each GEMM over three-term fp16 splits
        lowp = self.code != _lib.JC_F32 and not x3  # storage-type operands (the FP16 GEMM mode)

        def view(buf, width):  # a contiguous [tokens, width] view of a shared buffer
            return buf.view(-1)[: tokens_n * width].view(tokens_n, width)

        def operand(src, k):  # a GEMM's A operand: src itself, or (f16x3) its split [hi | hi | lo]
            if not x3:
                return src
            dst = view(b["x3"], 3 * k)
            chronos2.split_f16x3(src, dst)
            return dst

        def norm(wt):  # the pre-norm, in the GEMM operands' type
            if lowp:
                chronos2.rms_norm_lp(x, wt, b["hn_lp"], c.norm_eps)
                return b["hn_lp"]
            if x3:  # the norm writes the split itself
                y3 = view(b["x3"], 3 * d)
                chronos2.rms_norm_x3(x, wt, y3, c.norm_eps)
                return y3
            chronos2.rms_norm(x, wt, b["hn"], c.norm_eps)
            return b["hn"]

        def gemm(a, wt, out, flags=0):
            (chronos2.linear_lp if lowp or x3 else chronos2.linear)(a, wt, out, flags=flags)

        for lw in self.layers:
            for a in lw["attentions"]:
                hn = norm(a["norm"])
                # both attention cores read q|k|v and the gate in the storage type (fp32 arithmetic)
                lp_att = lowp
                qkv = view(b["big_lp"] if lp_att else b["big"], 3 * d)
                att = b["att_lp"] if lp_att else b["att"]
                gemm(hn, a["qkv"], qkv)
                g = None
                if a["gate"] is not None:
                    g = b["gate_lp"] if lp_att else b["gate"]
                    gemm(hn, a["gate"], g)
                if a["time"]:
                    timestral.time_attention(qkv, att, key_valid, known, pos, b["table"], g, rows, enc, ll, n, heads,
                                             dh, d)
                else:
                    timestral.variate_attention(qkv, att, key_valid, group_start, group_end, role, covariates, g, rows,
                                                enc, n, heads, dh, d)
                gemm(operand(att, d), a["wo"], x, chronos2.GEMM_ACCUMULATE)
            if not mlp:
                continue
            hn = norm(lw["mlp_norm"])
            up = view(b["big_lp"] if lowp else b["big"], 2 * f)
            act = b["act_lp"] if lowp else b["act"]
            gemm(hn, lw["up"], up)
            if x3:  # SwiGLU writes the down projection's split operand itself
                act = view(b["x3"], 3 * f)
                _lib.call("jc_swiglu", ctx.handle, p(up), p(act), tokens_n, f, _lib.JC_F16X3)
            else:
                _lib.call("jc_swiglu", ctx.handle, p(up), p(act), tokens_n, f, self.code if lowp else _lib.JC_F32)
            gemm(act, lw["down"], x, chronos2.GEMM_ACCUMULATE)

    def predict_block(self, inputs, observed, group, h: int, role=None, known_future=None, known_future_mask=None):
        """TimestralForward.predictBlock (TimestralForward.java:186-195): with buckets on, the block padded
        to its shared shape (leading empty patches, empty series of their own; neither is ever a valid
        key and positions count from each series' first observation, so the real rows' forecasts do
        not change), and the real rows' forecasts returned. See predict_exact."""
        if self.buckets:
            padded = bucketed(inputs, observed, group, h, role, known_future, known_future_mask, self.c.patch_size)
            if padded is not None:
                rows = np.asarray(inputs).shape[0]
                return self.predict_exact(*padded)[:rows]
        return self.predict_exact(inputs, observed, group, h, role, known_future, known_future_mask)

    def predict_exact(self, inputs, observed, group, h: int, role=None, known_future=None, known_future_mask=None):
        """TimestralModel.predict_block on one block, as CpuTimestral.predictBlock runs it
        (J/timestral/cpu/CpuTimestral.java:127-188): BlockLayout's window and masks on the host
        (block_window, jc_ts_block_layout), then on the device BlockPrep (jc_ts_prep), the forward and
        BlockPrep.finish (jc_ts_finish), so only the window goes up and the quantiles come down.
        inputs / observed [rows, t] (t a multiple of the patch), group [rows] with each series' rows
        contiguous, h forecast patches, role [rows] (0 TARGET, 1 PAST, 2 KNOWN) and the known
        covariates' future steps [rows, h*P] for a covariate block. Returns [rows, h*P, Q]
        quantiles. With plans, the whole block (uploads, prep, replay, finish, download) runs on the
        model's stream, so every launch and copy of it is ordered on that one stream."""
        import torch

        if self.plans is not None:
            with torch.cuda.stream(self._stream):
                return self._predict(inputs, observed, group, h, role, known_future, known_future_mask)
        return self._predict(inputs, observed, group, h, role, known_future, known_future_mask)

    def _predict(self, inputs, observed, group, h: int, role, known_future, known_future_mask):
        import torch

        c = self.c
        ps, q = c.patch_size, c.num_quantiles
        window, obs, cov = block_window(c, inputs, observed, role, known_future, known_future_mask, h)
        rows, t = np.asarray(inputs).shape
        wlen = window.shape[1]
        enc, cov_l, kv, known, pos = timestral.block_layout(
            observed, group, h, ps, role=role if cov else None, future_observed=known_future_mask if cov else None,
            covariate_enabled=c.covariate_enabled, attend_missing=c.attend_missing, block_size=c.block_size)
        if enc != wlen // ps or cov_l != cov:
            raise _lib.JitcastError(_lib.JC_EINVAL, "block layout and window disagree")
        gs, ge = chronos2.group_bounds(group)
        dev = self.dev
        up = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)  # noqa: E731
        ctx = chronos2.context(dev.index or 0)
        p = chronos2._ptr
        win_d = torch.from_numpy(np.ascontiguousarray(window, np.float32)).to(dev)
        obs_d = torch.from_numpy(np.ascontiguousarray(obs, np.uint8)).to(dev)
        known_d = up(known)
        tok = torch.empty(rows * enc, 2 * ps, dtype=torch.float32, device=dev)
        loc = torch.empty(rows, wlen, dtype=torch.float32, device=dev)
        scale = torch.empty(rows, wlen, dtype=torch.float32, device=dev)
        _lib.call("jc_ts_prep", ctx.handle, p(win_d), p(obs_d), rows, wlen, ps, p(known_d), c.minimum_scale,
                  int(c.use_asinh), p(tok), None, p(loc), p(scale))
        kv_d, pos_d, gs_d, ge_d = up(kv.reshape(-1)), up(pos.reshape(-1)), up(gs), up(ge)
        role_d = up(role) if cov else None
        if self.plans is not None:
            raw = self._forward_planned(tok, kv_d, known_d, pos_d, gs_d, ge_d, role_d, cov, rows, enc, h)
        else:
            raw = self.forward_raw(tok, kv_d, known_d, pos_d, gs_d, ge_d, role_d, cov, rows, enc, h)
        out = torch.empty(rows, h * ps, q, dtype=torch.float32, device=dev)
        widths = quantile_widths(c)
        ctx = chronos2.context(dev.index or 0)  # bound again: a capture above binds the context too
        _lib.call("jc_ts_finish", ctx.handle, p(raw), p(loc), p(scale), rows, wlen, t // ps, h, ps, q,
                  widths.ctypes.data, c.median_index, int(c.use_asinh), p(out))
        return out.cpu().numpy()


    def _forward_planned(self, tok, kv, known, pos, gs, ge, role, cov: bool, rows: int, enc: int, h: int):
        """The forward replayed from the plan of Shape(rows, encoder, horizon, covariates)
        (TimestralForward.predictExact's plans.run): the per-call inputs copied into the plan's buffers,
        then its captured forward; returns the plan's raw output. Runs on the model's stream, which
        predict_exact makes current."""
        shape = (rows, enc, h, bool(cov))

        def use(plan):
            b = plan.bufs
            b["tok"].copy_(tok)
            b["kv"].copy_(kv)
            b["known"].copy_(known)
            b["pos"].copy_(pos)
            b["gs"].copy_(gs)
            b["ge"].copy_(ge)
            if role is not None:
                b["role"].copy_(role)
            runtime.timed_replay(f"timestral.hip.profile shape={shape}", self.profile, plan.graph.launch)
            return b["raw"]

        return self.plans.run(shape, self._capture, use)

    def _capture(self, shape) -> "chronos2_model.ShapePlan":
        """TimestralForward.Plan's constructor: the shape's buffers, then the device forward captured
        into one hipGraph on the model's stream."""
        import torch

        rows, enc, h, cov = shape
        b = self._alloc(rows, enc, h, inputs=True)
        key = (rows << 40) | (enc << 20) | (h << 1) | int(cov)
        with torch.cuda.stream(self._stream):
            with plans_mod.capture(key, self.dev.index or 0) as box:
                self.forward_raw(b["tok"], b["kv"], b["known"], b["pos"], b["gs"], b["ge"], b["role"] if cov else None,
                                 cov, rows, enc, h, bufs=b)
        return chronos2_model.ShapePlan(box[0], b)

    def close(self) -> None:
        """Closes every cached plan (TimestralForward.close)."""
        if self.plans is not None:
            self.plans.close()


def bucket(x: int) -> int:
    """TimestralForward.bucket (TimestralForward.java:81-99): x itself up to 8, then the next multiple
    of a quarter of its power of two (9-16 in steps of 2, 17-32 in steps of 4, ...), so padding adds
    at most 25% and the number of shapes grows with the logarithm of the size."""
    if x <= 8:
        return x
    step = (1 << ((x - 1).bit_length() - 1)) // 4
    return (x + step - 1) // step * step


def bucketed(inputs, observed, group, h: int, role, known_future, known_future_mask, patch: int):
    """TimestralForward.bucketed (TimestralForward.java:197-232): the block padded to bucket(patches)
    patches (leading steps unobserved zeros) and bucket(rows) rows (each added row an empty target
    series of its own), as (inputs, observed, group, h, role, known_future, known_future_mask); None
    when the block already has a shared shape."""
    x = np.asarray(inputs, np.float32)
    r, t = x.shape
    patches = t // patch
    pad_patches, rows = bucket(patches), bucket(r)
    if pad_patches == patches and rows == r:
        return None
    lead, length = (pad_patches - patches) * patch, pad_patches * patch
    xi = np.zeros((rows, length), np.float32)
    ob = np.zeros((rows, length), bool)
    xi[:r, lead:lead + t] = x
    ob[:r, lead:lead + t] = np.asarray(observed, bool)
    g = np.asarray(group, np.int32)
    next_group = (int(g.max()) if g.size else 0) + 1
    grp = np.concatenate([g, np.arange(next_group, next_group + rows - r, dtype=np.int32)])
    rl = None if role is None else np.concatenate([np.asarray(role, np.int32), np.zeros(rows - r, np.int32)])
    kf = kfm = None
    if known_future is not None:
        f = np.asarray(known_future, np.float32)
        kf = np.zeros((rows, f.shape[1]), np.float32)
        kf[:r] = f
        kfm = np.zeros((rows, f.shape[1]), bool)
        kfm[:r] = np.asarray(known_future_mask, bool)
    return xi, ob, grp, h, rl, kf, kfm


FLOAT32_EPS = np.float32(np.finfo(np.float32).eps)


def block_window(c: TimestralConfig, inputs, observed, role=None, known_future=None, known_future_mask=None,
                 h: int = 1):
    """BlockLayout.of's window (BlockLayout.java:77-109): the context rows, plus the horizon's known
    future steps when the block runs the covariate path (role given, covariates enabled, some row not
    a TARGET). Returns (window float32 [rows, w], observed bool [rows, w], covariates)."""
    x = np.ascontiguousarray(inputs, dtype=np.float32)
    obs = np.ascontiguousarray(observed, dtype=bool)
    rows, t = x.shape
    if t % c.patch_size:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"context length {t} is not a multiple of the patch size")
    if h < 1:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"horizon patches must be >= 1, got {h}")
    cov = role is not None and c.covariate_enabled and bool(np.any(np.asarray(role) != 0))
    if not cov:
        return x, obs, False
    if h > c.block_size:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"a block with covariates decodes at most {c.block_size} patches")
    w = t + h * c.patch_size
    win = np.zeros((rows, w), np.float32)
    ob = np.zeros((rows, w), bool)
    win[:, :t], ob[:, :t] = x, obs
    if known_future is not None:
        win[:, t:] = np.asarray(known_future, np.float32)[:, : h * c.patch_size]
        ob[:, t:] = np.asarray(known_future_mask, bool)[:, : h * c.patch_size]
    return win, ob, True


def _causal_patch_loc_scale(x, obs, patch, minimum_scale):
    """Scaler.causalPatchLocScale (Scaler.java:40-64), all rows at once: a running weighted mean and
    Welford M2 in double; at each patch end, loc = mean and scale = max(sqrt(M2 / max(max(w,1)-1,1)),
    minimum) rounded to float for the patch's steps."""
    rows, t = x.shape
    ms = np.float64(np.float32(minimum_scale))  # the config's float, widened as Java widens it
    xd = x.astype(np.float64)
    wd = obs.astype(np.float64)
    cum_w = np.zeros(rows)
    cum_x = np.zeros(rows)
    m2 = np.zeros(rows)
    prev = np.zeros(rows)
    loc = np.empty((rows, t), np.float32)
    scale = np.empty((rows, t), np.float32)
    for i in range(t):
        cum_w += wd[:, i]
        cum_x += wd[:, i] * xd[:, i]
        mean = cum_x / np.maximum(cum_w, 1.0)
        m2 += (xd[:, i] - prev) * (xd[:, i] - mean) * wd[:, i]
        prev = mean
        if i % patch == patch - 1:
            var = m2 / np.maximum(np.maximum(cum_w, 1.0) - 1.0, 1.0)
            loc[:, i - patch + 1: i + 1] = mean.astype(np.float32)[:, None]
            scale[:, i - patch + 1: i + 1] = np.maximum(np.sqrt(var), ms).astype(np.float32)[:, None]
    return loc, scale


def _instance_norm(x, obs, minimum_scale):
    """Scaler.instanceNorm (Scaler.java:87-110) for one row: (loc, scale, binary) in float from sums
    in double; a row of observed 0/1 values gives (0, 1, binary)."""
    n = max(float(np.count_nonzero(obs)), 1.0)
    loc = np.float32(np.sum(x[obs].astype(np.float64)) / n)
    d = np.where(obs, x - loc, np.float32(0)).astype(np.float32)
    ss = float(np.sum(d.astype(np.float64) ** 2))
    scale = max(np.float32(np.sqrt(np.float32(ss / n))), np.float32(minimum_scale))
    binary = bool(np.all((x == 0) | (x == 1) | ~obs)) and bool(np.any(obs))
    return (np.float32(0), np.float32(1), True) if binary else (loc, np.float32(scale), False)


def _asinh(v):
    a = np.abs(v.astype(np.float64))
    r = np.log(a + np.sqrt(a * a + 1.0))
    return np.where(v < 0, -r, r).astype(np.float32)


def block_prep(c: TimestralConfig, window, obs, known_rows):
    """BlockPrep.of (BlockPrep.java:40-75): per row the causal patch scaler (whole-row instance norm
    for known covariates), the scaled window (0 where unobserved, arcsinh unless a binary covariate)
    and the embedding input of every encoder token [values, missing flags]. Returns (tokens
    [rows*enc, 2P], scaled, loc, scale [rows, w])."""
    ps = c.patch_size
    rows, w = window.shape
    enc = w // ps
    loc, scale = _causal_patch_loc_scale(window, obs, ps, c.minimum_scale)
    asinh_row = np.full(rows, c.use_asinh)
    for i in np.flatnonzero(np.asarray(known_rows, bool)):
        lo, sc, binary = _instance_norm(window[i], obs[i], c.minimum_scale)
        loc[i], scale[i] = lo, sc
        asinh_row[i] = c.use_asinh and not binary
    v = ((window - loc) / np.maximum(scale, FLOAT32_EPS)).astype(np.float32)
    v = np.where(asinh_row[:, None], _asinh(v), v)
    scaled = np.where(obs, v, np.float32(0)).astype(np.float32)
    tok = np.empty((rows, enc, 2 * ps), np.float32)
    tok[:, :, :ps] = scaled.reshape(rows, enc, ps)
    tok[:, :, ps:] = np.where(obs, np.float32(0), np.float32(1)).reshape(rows, enc, ps)
    return tok.reshape(rows * enc, 2 * ps), scaled, loc, scale


def _softplus(x):
    xd = x.astype(np.float64)
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(xd, 20.0))).astype(np.float32)).astype(np.float32)


def quantile_widths(c: TimestralConfig):
    """Quantiles' per-level widthFactor * dp (Quantiles.java:30-41): the gap to the next level inward,
    rounded to float, times the float width factor. float32 [Q]."""
    knots = np.asarray(c.quantiles, np.float64)
    q, med = len(knots), c.median_index
    width = np.zeros(q, np.float32)
    for i in range(q):
        width[i] = np.float32(knots[i] - knots[i - 1] if i > med else knots[i + 1] - knots[i] if i < med else 0.0)
    return (np.float32(c.quantile_width_factor) * width).astype(np.float32)


def quantile_map(c: TimestralConfig, raw):
    """Quantiles.apply (Quantiles.java:52-77) on every row of raw [..., Q]: the median kept, each
    level above it the median plus the running sum of widthFactor*dp*softplus(raw), each level
    below minus it, clamped to the finite float range. Widths rounded to float as the reference's
    tensor holds them."""
    q, med = c.num_quantiles, c.median_index
    width = quantile_widths(c)
    raw = np.asarray(raw, np.float32)
    out = np.empty_like(raw)
    m = raw[..., med]
    big = np.float32(np.finfo(np.float32).max)
    up = np.zeros(m.shape, np.float32)
    for i in range(med + 1, q):
        up = (up + width[i] * _softplus(raw[..., i])).astype(np.float32)
        out[..., i] = np.clip(m + up, -big, big)
    down = np.zeros(m.shape, np.float32)
    for i in range(med - 1, -1, -1):
        down = (down + width[i] * _softplus(raw[..., i])).astype(np.float32)
        out[..., i] = np.clip(m - down, -big, big)
    out[..., med] = np.clip(m, -big, big)
    return out


def _clamp_non_finite(v):
    """Scaler.clampNonFinite (Scaler.java:118-130) over the last axis: +inf to the finite max, -inf
    to the finite min, 0 where no finite value exists."""
    fin = np.isfinite(v)
    vmax = np.where(fin, v, -np.inf).max(axis=-1, keepdims=True)
    vmin = np.where(fin, v, np.inf).min(axis=-1, keepdims=True)
    x = np.where(v == np.inf, vmax, np.where(v == -np.inf, vmin, v))
    return np.where(np.isinf(x), np.float32(0), x).astype(np.float32)


def block_finish(c: TimestralConfig, raw, loc, scale, ll: int, h: int):
    """BlockPrep.finish (BlockPrep.java:77-101): the quantile map on raw [rows*h, P*Q] (steps
    P-major, Q levels contiguous), then each step denormalized with the frame of the last context
    patch (sinh when the scaler used arcsinh; float multiply then add) and non-finite values clamped.
    Returns [rows, h*P, Q]."""
    ps, q = c.patch_size, c.num_quantiles
    rows = loc.shape[0]
    v = quantile_map(c, np.asarray(raw, np.float32).reshape(rows, h * ps, q))
    a_loc = loc[:, (ll - 1) * ps][:, None, None]
    a_scale = scale[:, (ll - 1) * ps][:, None, None]
    with np.errstate(over="ignore"):
        if c.use_asinh:
            v = np.sinh(v.astype(np.float64)).astype(np.float32)
        out = (v * a_scale).astype(np.float32) + a_loc
    return _clamp_non_finite(out.astype(np.float32))
