"""Timestral attention stages on libjitcast_hip, with the reference's per-layer contract.

Each function takes the arguments of the reference kernel it replaces, as torch tensors resident
on the GPU, and launches on torch's current stream:

  time_attention   TimestralKernels.rope + timeAttention + gate
                   (J/timestral/tornado/TimestralKernels.java:77-78, 114-115, 573), fused
  variate_attention  TimestralKernels.variateAttention + gate (TimestralKernels.java:290-292, 573)
  gate             TimestralKernels.gate (TimestralKernels.java:572-578)
  rope_table       the host-built table of TimestralForward.Plan.run (TimestralForward.java:599-610)
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .chronos2 import _dtype_code, _ptr
from .runtime import context


def rope_table(enc: int, n: int, dh: int, rope_dim: int, theta: float = 10000.0) -> np.ndarray:
    """[(enc + n), dh] float32: row p rotates by position p - enc (cos half, then sin half)."""
    out = np.empty((enc + n, dh), dtype=np.float32)
    _lib.call("jc_ts_rope_table", enc, n, dh, rope_dim, ctypes.c_float(theta), out.ctypes.data_as(ctypes.c_void_p))
    return out


def time_attention(qkv, out, key_valid, known, pos, table, gate, rows: int, enc: int, ll: int, n: int, heads: int,
                   dh: int, d: int) -> None:
    """One Timestral time-attention sublayer: RoPE at pos, masked softmax(q.k/sqrt(dh)) v, and
    out *= sigmoid(gate) when gate is given.

    qkv [rows*n, 3*d] and out (and gate) [rows*n, d]: float32, bfloat16 or float16, all the same;
    key_valid int32 [rows*enc]; known int32 [rows] or None; pos int32 [rows*n] (table rows) or None;
    table float32 [(enc+n), dh] or None.
    """
    dt = _dtype_code(qkv)
    if _dtype_code(out) != dt or (gate is not None and _dtype_code(gate) != dt):
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "qkv, out and gate must have the same dtype")
    ctx = context(qkv.device.index or 0)
    _lib.call("jc_ts_time_attention", ctx.handle, _ptr(qkv), _ptr(out), _ptr(key_valid), _ptr(known), _ptr(pos),
              _ptr(table), _ptr(gate), rows, enc, ll, n, heads, dh, d, dt)


def variate_attention(qkv, out, key_valid, group_start, group_end, role, covariates: bool, gate, rows: int,
                      enc: int, n: int, heads: int, dh: int, d: int) -> None:
    """Attention across the rows of each series per slot (TimestralKernels.variateAttention), scaled
    by 1/sqrt(dh), under BlockLayout.variateAllowed; out *= sigmoid(gate) when gate is given.

    qkv [rows*n, 3*d] and out (and gate) [rows*n, d] float32, bfloat16 or float16 (all the same; fp32
    arithmetic); key_valid int32 [rows*enc];
    group_start/group_end int32 [rows] (contiguous groups); role int32 [rows] or None.
    """
    dt = _dtype_code(qkv)
    if _dtype_code(out) != dt or (gate is not None and _dtype_code(gate) != dt):
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "qkv, out and gate must have the same dtype")
    ctx = context(qkv.device.index or 0)
    _lib.call("jc_ts_variate_attention", ctx.handle, _ptr(qkv), _ptr(out), _ptr(key_valid), _ptr(group_start),
              _ptr(group_end), _ptr(role), int(bool(covariates)), _ptr(gate), rows, enc, n, heads, dh, d, dt)


def block_layout(observed, group, h: int, patch: int, role=None, future_observed=None, covariate_enabled=True,
                 attend_missing=True, block_size: int = 1 << 30):
    """BlockLayout.of (J/timestral/BlockLayout.java:77-148) on the host.

    observed [rows, t] bool/0-1; group [rows]; role [rows] or None; future_observed [rows, h*patch]
    or None. Returns (enc, covariates, key_valid [rows, enc], known [rows], pos [rows, enc+h]) with
    pos holding table rows (position + enc) for time_attention.
    """
    obs = np.ascontiguousarray(observed, dtype=np.uint8)
    rows, t = obs.shape
    g = np.ascontiguousarray(group, dtype=np.int32)
    r = None if role is None else np.ascontiguousarray(role, dtype=np.int32)
    fut = None if future_observed is None else np.ascontiguousarray(future_observed, dtype=np.uint8)
    enc_max = t // patch + h
    kv = np.zeros(rows * enc_max, np.int32)
    known = np.zeros(rows, np.int32)
    pos = np.zeros(rows * (enc_max + h), np.int32)
    enc, cov = ctypes.c_int(), ctypes.c_int()

    def p(a):
        return ctypes.c_void_p(0) if a is None else a.ctypes.data_as(ctypes.c_void_p)

    _lib.call("jc_ts_block_layout", p(obs), p(fut), p(g), p(r), rows, t, patch, h, int(bool(covariate_enabled)),
              int(bool(attend_missing)), block_size, ctypes.byref(enc), ctypes.byref(cov), p(kv), p(known), p(pos))
    e = enc.value
    return e, bool(cov.value), kv[: rows * e].reshape(rows, e), known, pos[: rows * (e + h)].reshape(rows, e + h)


def gate(att, g) -> None:
    """att *= sigmoid(g), in place (TimestralKernels.gate)."""
    dt = _dtype_code(att)
    if _dtype_code(g) != dt or g.numel() < att.numel():
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "att and g must have the same dtype and size")
    ctx = context(att.device.index or 0)
    _lib.call("jc_ts_gate", ctx.handle, _ptr(att), _ptr(g), att.numel(), dt)
