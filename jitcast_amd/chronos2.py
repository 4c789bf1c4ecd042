"""Chronos-2 attention stages on libjitcast_hip, with the reference's per-layer contract.

Each function takes the arguments of the reference kernel it replaces, as torch tensors resident
on the GPU, and launches on torch's current stream:

  time_attention   Chronos2Kernels.rope + Chronos2Kernels.timeAttention
                   (J/chronos2/tornado/Chronos2Kernels.java:93-94, 130-131), fused
  group_attention  Chronos2Kernels.groupAttention (Chronos2Kernels.java:473-474)
  rope_table       the host-built table of Chronos2Forward.Plan.run (Chronos2Forward.java:465-474)
  live_mask, group_order, group_bounds   ModelLayout.java:104-114, Chronos2Forward.java:178-194, 475-489
  linear           Kernels.gemm and its flags (J/tornado/Kernels.java:50-103), as Chronos2Forward.Plan.gemm
                   calls it (Chronos2Forward.java:312-369)
  rms_norm         Kernels.rmsNorm (Kernels.java:800-829)
  layer            one encoder layer: the per-layer stage of Chronos2Forward.Plan (Chronos2Forward.java:258-286)
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

    qkv [rows*n, 3*inner] and out [rows*n, inner] float32, bfloat16 or float16 (both the same; fp32
    arithmetic); group_start/group_end: int32 [rows] device tensors (see group_bounds); groups contiguous.
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


GEMM_BIAS, GEMM_ACCUMULATE, GEMM_SILU, GEMM_RELU = 1, 2, 4, 16


def _f32(t, name):
    if str(t.dtype) != "torch.float32":
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, f"{name} must be float32")


def linear(a, w, c, bias=None, flags: int = 0, m: int | None = None, n: int | None = None, k: int | None = None,
           lda: int | None = None, ldc: int | None = None) -> None:
    """c (+)= act(a . w^T + bias) on torch's current stream; w is [n, k] (PyTorch's Linear layout).

    flags: GEMM_ACCUMULATE, GEMM_RELU, GEMM_SILU (GEMM_BIAS is implied by a bias). Sizes default to
    the tensors' shapes: a [m, k] (row stride lda), c [m, n] (row stride ldc).
    """
    for t, nm in ((a, "a"), (w, "w"), (c, "c")):
        _f32(t, nm)
    m = a.shape[0] if m is None else m
    n = w.shape[0] if n is None else n
    k = w.shape[1] if k is None else k
    lda = a.stride(0) if lda is None else lda
    ldc = c.stride(0) if ldc is None else ldc
    ctx = context(a.device.index or 0)
    _lib.call("jc_linear", ctx.handle, _ptr(a), lda, _ptr(w), _ptr(bias), _ptr(c), ldc, m, n, k, flags)


def rms_norm(x, w, y, eps: float) -> None:
    """y = x * (1 / sqrt(mean(x^2) + eps)) * w per row; x, y [rows, d] float32 (may be the same tensor)."""
    _f32(x, "x")
    _f32(y, "y")
    ctx = context(x.device.index or 0)
    rows, d = x.shape
    _lib.call("jc_rms_norm", ctx.handle, _ptr(x), _ptr(w), _ptr(y), rows, d, ctypes.c_float(eps))


class LayerWeights(ctypes.Structure):
    """jc_c2_layer_weights: device pointers of one encoder layer (Chronos2Packed.Layer)."""

    _fields_ = [(name, ctypes.c_void_p) for name in (
        "time_norm", "time_qkv", "time_qkv_bias", "time_o", "time_o_bias",
        "group_norm", "group_qkv", "group_qkv_bias", "group_o", "group_o_bias",
        "mlp_norm", "wi", "wi_bias", "wo", "wo_bias")]

    @classmethod
    def of(cls, tensors: dict) -> "LayerWeights":
        """From a dict of float32 device tensors keyed by field name (missing biases are NULL)."""
        lw = cls()
        for name, _ in cls._fields_:
            t = tensors.get(name)
            setattr(lw, name, t.data_ptr() if t is not None else None)
        return lw


def layer_workspace_bytes(rows: int, n: int, d: int, inner: int, dff: int, dtype: int = _lib.JC_F32) -> int:
    return int(_lib.lib().jc_c2_layer_workspace_bytes(rows, n, d, inner, dff, dtype))


def layer(x, weights: dict, live, table, group_start, group_end, workspace, rows: int, n: int, d: int, heads: int,
          dh: int, dff: int, eps: float, dtype: int = _lib.JC_F32) -> None:
    """One Chronos-2 encoder layer in place on x [rows*n, d] float32 (see include/jitcast_hip.h).

    dtype JC_F32: fp32 weights. JC_BF16 / JC_F16: the weight matrices in that type (to_lp converts
    them), norm weights and biases fp32; GEMMs and time attention in the storage type with fp32
    accumulation, the residual stream fp32. JC_F16X3: the weight matrices as fp16 [n, 3k] W-operand
    splits (split_f16x3 with weights=True); each GEMM product within about 2^-20 |a w| +
    2^-25 (|a| + |w|), fp32 accumulation and outputs."""
    _f32(x, "x")
    ctx = context(x.device.index or 0)
    lw = LayerWeights.of(weights)
    _lib.call("jc_c2_layer", ctx.handle, _ptr(x), ctypes.byref(lw), _ptr(live), _ptr(table), _ptr(group_start),
              _ptr(group_end), _ptr(workspace), rows, n, d, heads, dh, dff, ctypes.c_float(eps), dtype)


# JC_C2_LAYER_STATIC_BYTES: the device scratch jc_c2_layer_static runs in
LAYER_STATIC_BYTES = 64 << 20


def layer_static(x, weights: dict, live, table, group_start, group_end, rows: int, n: int, d: int, heads: int,
                 dh: int, dff: int, eps: float, dtype: int = _lib.JC_F32) -> None:
    """layer() without a workspace: jc_c2_layer_static runs the layer in the library's own device
    scratch (LAYER_STATIC_BYTES per GPU) and allocates nothing; a call whose workspace would exceed it
    raises JitcastArgumentError. Calls that overlap on one GPU race on that scratch."""
    _f32(x, "x")
    ctx = context(x.device.index or 0)
    lw = LayerWeights.of(weights)
    _lib.call("jc_c2_layer_static", ctx.handle, _ptr(x), ctypes.byref(lw), _ptr(live), _ptr(table),
              _ptr(group_start), _ptr(group_end), rows, n, d, heads, dh, dff, ctypes.c_float(eps), dtype)


def linear_lp(a, w, c, bias=None, flags: int = 0, m: int | None = None, n: int | None = None, k: int | None = None,
              lda: int | None = None, ldc: int | None = None) -> None:
    """c (+)= act(a . w^T + bias): a and w bfloat16 or float16 (the same), c float32 or that type
    (no GEMM_ACCUMULATE then); fp32 accumulation (Kernels.gemmHalf's contract)."""
    dt = _dtype_code(a)
    if dt == _lib.JC_F32 or _dtype_code(w) != dt:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "a and w must both be bfloat16 or both float16")
    m = a.shape[0] if m is None else m
    n = w.shape[0] if n is None else n
    k = w.shape[1] if k is None else k
    lda = a.stride(0) if lda is None else lda
    ldc = c.stride(0) if ldc is None else ldc
    ctx = context(a.device.index or 0)
    _lib.call("jc_linear_lp", ctx.handle, _ptr(a), lda, _ptr(w), _ptr(bias), _ptr(c), ldc, m, n, k, flags, dt,
              _dtype_code(c))


def rms_norm_lp(x, w, y, eps: float) -> None:
    """y (bfloat16 or float16) = rmsNorm(x) with x float32 [rows, d]."""
    _f32(x, "x")
    ctx = context(x.device.index or 0)
    rows, d = x.shape
    _lib.call("jc_rms_norm_lp", ctx.handle, _ptr(x), _ptr(w), _ptr(y), rows, d, ctypes.c_float(eps), _dtype_code(y))


def rms_norm_x3(x, w, y3, eps: float) -> None:
    """y3 float16 [rows, 3d] = the split [hi | hi | lo] of rmsNorm(x), x float32 [rows, d]
    (jc_rms_norm_lp with JC_F16X3): the norm and jc_split_f16x3 in one pass."""
    _f32(x, "x")
    rows, d = x.shape
    if y3.dim() != 2 or tuple(y3.shape) != (rows, 3 * d) or _dtype_code(y3) != _lib.JC_F16:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "rms_norm_x3: y3 must be float16 [rows, 3d]")
    ctx = context(x.device.index or 0)
    _lib.call("jc_rms_norm_lp", ctx.handle, _ptr(x), _ptr(w), _ptr(y3), rows, d, ctypes.c_float(eps), _lib.JC_F16X3)


def split_f16x3(src, dst, weights: bool = False) -> None:
    """dst float16 [rows, 3k] = the three-term split of src float32 [rows, k] (jc_split_f16x3):
    [hi | hi | lo] per row, or [hi | lo | hi] with weights, hi = fp16(v) saturated, lo = fp16(v - hi)."""
    _f32(src, "src")
    if src.dim() != 2 or dst.dim() != 2 or dst.shape[0] != src.shape[0] or dst.shape[1] != 3 * src.shape[1]:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "split_f16x3: src [rows, k] and dst [rows, 3k]")
    if _dtype_code(dst) != _lib.JC_F16:
        raise _lib.JitcastArgumentError(_lib.JC_EINVAL, "split_f16x3: dst must be float16")
    ctx = context(src.device.index or 0)
    _lib.call("jc_split_f16x3", ctx.handle, _ptr(src), src.stride(0), _ptr(dst), src.shape[0], src.shape[1],
              1 if weights else 0)


def to_lp(src, dst) -> None:
    """dst (bfloat16 or float16) = src (float32) rounded, saturated to the type's finite range."""
    _f32(src, "src")
    ctx = context(src.device.index or 0)
    _lib.call("jc_to_lp", ctx.handle, _ptr(src), _ptr(dst), ctypes.c_int64(src.numel()), _dtype_code(dst))


def prep(series, future, order, rows: int, context_length: int, patch: int, h: int, nreg: int,
         time_scale: float, arcsinh: bool):
    """ModelLayout.of's cut and live mask plus ModelPrep.of on the device (jc_c2_prep): series
    [rows, T] fp32 on the GPU (NaN where missing), future [rows, <= h*patch] or None, order int32
    [rows] or None (output row i is input row order[i]). Returns (tokens [rows*(nc+h), 3*patch],
    loc [rows], scale [rows], live [rows*(nc+nreg+h)] int32, nc), all on the series' device."""
    import torch

    ctx = context(series.device.index or 0)
    t = int(series.shape[1])
    kept = min(t, context_length)
    nc = (kept + patch - 1) // patch
    dev = series.device
    tok = torch.empty(rows * (nc + h), 3 * patch, dtype=torch.float32, device=dev)
    loc = torch.empty(rows, dtype=torch.float32, device=dev)
    scale = torch.empty(rows, dtype=torch.float32, device=dev)
    live = torch.empty(rows * (nc + nreg + h), dtype=torch.int32, device=dev)
    fs = int(future.shape[1]) if future is not None else 0
    ldf = int(future.stride(0)) if future is not None else 0
    _lib.call("jc_c2_prep", ctx.handle, _ptr(series), ctypes.c_int64(series.stride(0)), t, _ptr(future),
              ctypes.c_int64(ldf), fs, _ptr(order), rows, context_length, patch, h, nreg, ctypes.c_float(time_scale),
              int(bool(arcsinh)), _ptr(tok), _ptr(loc), _ptr(scale), _ptr(live))
    return tok, loc, scale, live, nc


def finish(raw, loc, scale, order, rows: int, h: int, q: int, patch: int, arcsinh: bool, out) -> None:
    """ModelPrep.finish on the device (jc_c2_finish): out [rows, q, h*patch] (row order[i] of out
    from row i of raw [rows*h, q*patch]) = sinh(raw) * scale + loc."""
    ctx = context(raw.device.index or 0)
    _lib.call("jc_c2_finish", ctx.handle, _ptr(raw), _ptr(loc), _ptr(scale), _ptr(order), rows, h, q, patch,
              int(bool(arcsinh)), _ptr(out))
