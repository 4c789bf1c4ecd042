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

The host ends (BlockLayout.of through jc_ts_block_layout, BlockPrep, the quantile head's
monotone map) stay on the host, as in the reference.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _lib, chronos2, timestral

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

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    @property
    def rope_dim(self) -> int:
        return int(self.head_dim * self.rope_partial_factor)

    @property
    def num_quantiles(self) -> int:
        return len(self.quantiles)


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
    """The Timestral block forward on one GPU, fp32 (the reference's FP32-exact default): weights
    uploaded once, per-shape buffers kept for the last shape, one call per block."""

    def __init__(self, c: TimestralConfig, weights: dict, device: int = 0):
        import torch

        self.c = c
        self.dev = torch.device("cuda", device)
        t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)  # noqa: E731
        self.w = {k: t(v) for k, v in weights.items() if k != "layers"}
        self.layers = [{"attentions": [{k: (a[k] if k == "time" else t(a[k])) for k in a} for a in lw["attentions"]],
                        "mlp_norm": t(lw["mlp_norm"]), "up": t(lw["up"]), "down": t(lw["down"])}
                       for lw in weights["layers"]]
        self._bufs = {}

    def _buffers(self, rows: int, enc: int, h: int):
        import torch

        key = (rows, enc, h)
        if key not in self._bufs:
            self._bufs.clear()
            c = self.c
            n, d, f = enc + h, c.d_model, c.mlp_hidden_dim
            tokens = rows * n
            e = lambda *s: torch.empty(*s, dtype=torch.float32, device=self.dev)  # noqa: E731
            self._bufs[key] = {
                "emb": e(rows * enc, d), "scratch": e(max(rows * enc, rows * h), 4 * d), "x": e(tokens, d),
                "hn": e(tokens, d), "big": e(tokens, max(3 * d, 2 * f)), "att": e(tokens, d), "gate": e(tokens, d),
                "act": e(tokens, f), "y": e(tokens, d), "dec": e(rows * h, d),
                "raw": e(rows * h, c.patch_size * c.num_quantiles),
                "table": torch.from_numpy(timestral.rope_table(enc, n, c.head_dim, c.rope_dim, c.rope_theta)).to(self.dev),
            }
        return self._bufs[key]

    def forward_raw(self, tokens, key_valid, known, pos, group_start, group_end, role, covariates: bool, rows: int,
                    enc: int, h: int):
        """The device forward from the patch tokens (torch [rows*enc, 2P] on the GPU) to the head's
        raw outputs [rows*h, P*Q] on the GPU. key_valid [rows*enc], known [rows] (or None), pos
        [rows*(enc+h)] table rows from jc_ts_block_layout, group_start / group_end [rows] and role
        [rows] (or None) as int32 device tensors; rows of a series contiguous."""
        c = self.c
        n, d, f, heads, dh = enc + h, c.d_model, c.mlp_hidden_dim, c.num_heads, c.head_dim
        ll = enc - h if covariates else enc
        tokens_n = rows * n
        b = self._buffers(rows, enc, h)
        w = self.w
        ctx = chronos2.context(self.dev.index or 0)
        p = chronos2._ptr
        _lib.call("jc_ts_residual", ctx.handle, p(tokens), rows * enc, 2 * c.patch_size, p(w["embed_hidden_w"]),
                  p(w.get("embed_hidden_b")), p(w["embed_output_w"]), p(w.get("embed_output_b")),
                  p(w["embed_residual_w"]), p(w.get("embed_residual_b")), 4 * d, d, p(b["scratch"]), p(b["emb"]))
        _lib.call("jc_ts_assemble", ctx.handle, p(b["emb"]), p(w["query"]), p(b["x"]), rows, enc, n, d)
        x, hn, big, att = b["x"], b["hn"], b["big"], b["att"]
        # q|k|v and the MLP's up projection share one buffer, each a contiguous [tokens, width] view
        qkv = big.view(-1)[: tokens_n * 3 * d].view(tokens_n, 3 * d)
        up = big.view(-1)[: tokens_n * 2 * f].view(tokens_n, 2 * f)
        for lw in self.layers:
            for a in lw["attentions"]:
                chronos2.rms_norm(x, a["norm"], hn, c.norm_eps)
                chronos2.linear(hn, a["qkv"], qkv)
                g = None
                if a["gate"] is not None:
                    chronos2.linear(hn, a["gate"], b["gate"])
                    g = b["gate"]
                if a["time"]:
                    timestral.time_attention(qkv, att, key_valid, known, pos, b["table"], g, rows, enc, ll, n, heads,
                                             dh, d)
                else:
                    timestral.variate_attention(qkv, att, key_valid, group_start, group_end, role, covariates, g, rows,
                                                enc, n, heads, dh, d)
                chronos2.linear(att, a["wo"], x, flags=chronos2.GEMM_ACCUMULATE)
            chronos2.rms_norm(x, lw["mlp_norm"], hn, c.norm_eps)
            chronos2.linear(hn, lw["up"], up)
            _lib.call("jc_swiglu", ctx.handle, p(up), p(b["act"]), tokens_n, f, _lib.JC_F32)
            chronos2.linear(b["act"], lw["down"], x, flags=chronos2.GEMM_ACCUMULATE)
        chronos2.rms_norm(x, w["out_norm"], b["y"], c.norm_eps)
        _lib.call("jc_ts_gather_decoder", ctx.handle, p(b["y"]), p(b["dec"]), rows, enc, n, h, d)
        _lib.call("jc_ts_residual", ctx.handle, p(b["dec"]), rows * h, d, p(w["head_hidden_w"]), None,
                  p(w["head_output_w"]), None, p(w["head_residual_w"]), None, 4 * d, c.patch_size * c.num_quantiles,
                  p(b["scratch"]), p(b["raw"]))
        return b["raw"]
