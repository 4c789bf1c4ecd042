"""Chronos-2 attention stages on libjitcast_hip, with the reference's per-layer contract.

Each function takes the arguments of the reference kernel it replaces, as torch tensors resident
on the GPU, and launches on torch's current stream:

  time_attention   Chronos2Kernels.rope + Chronos2Kernels.timeAttention
                   (J/chronos2/tornado/Chronos2Kernels.java:93-94, 130-131), fused
  rope_table       the host-built table of Chronos2Forward.Plan.run (Chronos2Forward.java:465-474)
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
