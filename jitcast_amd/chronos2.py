"""Chronos-2 attention stages on libjitcast_hip, with the reference's per-layer contract.

Each function takes the arguments of the reference kernel it replaces, as torch tensors resident
on the GPU, and launches on torch's current stream:

  time_attention   Chronos2Kernels.rope + Chronos2Kernels.timeAttention
                   (J/chronos2/tornado/Chronos2Kernels.java:93-94, 130-131), fused
  group_attention  Chronos2Kernels.groupAttention (Chronos2Kernels.java:473-474)
  rope_table       the host-built table of Chronos2Forward.Plan.run (Chronos2Forward.java:465-474)
  live_mask, group_order, group_bounds   ModelLayout.java:104-114, Chronos2Forward.java:178-194, 475-489
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .runtime import context

DTYPES = {"float32": _lib.JC_F32, "bfloat16": _lib.JC_BF16, "float16": _lib.JC_F16}


def _dtype_code(t) -> int:
    name = str(t.dtype).replace("torch.", "")
    if name not in DTYPES:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"unsupported dtype {t.dtype}")
    return DTYPES[name]


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def rope_table(n: int, dh: int, theta: float = 10000.0) -> np.ndarray:
    """[n, dh] float32: cos((float)p * invFreq[e]) for e < dh/2, then sin (built on the host)."""
    out = np.empty((n, dh), dtype=np.float32)
    _lib.call("jc_c2_rope_table", n, dh, ctypes.c_float(theta), out.ctypes.data_as(ctypes.c_void_p))
    return out


def time_attention(qkv, out, live, rows: int, n: int, heads: int, dh: int, inner: int, table=None) -> None:
    """out[(r*n+t)*inner + h*dh + e] = softmax over live keys of RoPE(q).RoPE(k), times v.

    qkv [rows*n, 3*inner] and out [rows*n, inner] are float32, bfloat16 or float16 (both the same);
    live [rows*n] int32; table [n, dh] float32 or None when qkv is already rotated.
    """
    dt = _dtype_code(qkv)
    if _dtype_code(out) != dt:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "qkv and out must have the same dtype")
    ctx = context(qkv.device.index or 0)
    _lib.call("jc_c2_time_attention", ctx.handle, _ptr(qkv), _ptr(out), _ptr(live), _ptr(table),
              rows, n, heads, dh, inner, dt)


def group_attention(qkv, out, live, group_start, group_end, rows: int, n: int, heads: int, dh: int,
                    inner: int) -> None:
    """Attention across the rows of each group at every slot (Chronos2Kernels.groupAttention).

    group_start/group_end: int32 [rows] device tensors (see group_bounds); groups contiguous.
    """
    dt = _dtype_code(qkv)
    if _dtype_code(out) != dt:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "qkv and out must have the same dtype")
    ctx = context(qkv.device.index or 0)
    _lib.call("jc_c2_group_attention", ctx.handle, _ptr(qkv), _ptr(out), _ptr(live), _ptr(group_start),
              _ptr(group_end), rows, n, heads, dh, inner, dt)


def live_mask(window: np.ndarray, nc: int, patch: int, reg: int, h: int) -> np.ndarray:
    """ModelLayout's live mask [rows, nc+reg+h] int32 from the NaN-padded window [rows, nc*patch]."""
    w = np.ascontiguousarray(window, dtype=np.float32)
    rows = w.shape[0]
    out = np.empty((rows, nc + reg + h), np.int32)
    _lib.call("jc_c2_live", w.ctypes.data_as(ctypes.c_void_p), rows, nc, patch, reg, h,
              out.ctypes.data_as(ctypes.c_void_p))
    return out


def group_order(group) -> np.ndarray | None:
    """Row order making groups contiguous (Chronos2Forward.groupOrder); None if already contiguous."""
    g = np.ascontiguousarray(group, dtype=np.int32)
    order = np.empty(len(g), np.int32)
    ident = ctypes.c_int()
    _lib.call("jc_c2_group_order", g.ctypes.data_as(ctypes.c_void_p), len(g), order.ctypes.data_as(ctypes.c_void_p),
              ctypes.byref(ident))
    return None if ident.value else order


def group_bounds(group) -> tuple[np.ndarray, np.ndarray]:
    """Per-row [start, end) of each row's (contiguous) group; raises if a group is split."""
    g = np.ascontiguousarray(group, dtype=np.int32)
    start = np.empty(len(g), np.int32)
    end = np.empty(len(g), np.int32)
    _lib.call("jc_c2_group_bounds", g.ctypes.data_as(ctypes.c_void_p), len(g), start.ctypes.data_as(ctypes.c_void_p),
              end.ctypes.data_as(ctypes.c_void_p))
    return start, end
