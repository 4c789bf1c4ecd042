"""Independent float64 brute-force restatements used to pin the C oracle on small shapes.

Written from the reference's semantics (not from the oracle's code), vectorised with numpy so that
the two implementations share no structure: RoPE tables and rotated q/k follow the reference's
float32 rounding (CpuChronos2.java:102-111, 215-228), everything after is float64.
"""
from __future__ import annotations

import numpy as np


def inv_freq(dh: int, theta: float = 10000.0, rope_dim: int | None = None) -> np.ndarray:
    rot = dh if rope_dim is None else rope_dim
    f = np.zeros(dh // 2, np.float32)
    i = np.arange(rot // 2)
    ex = (np.float32(2) * i.astype(np.float32)) / np.float32(rot)  # float division, as (float)(2i)/(float)dh
    f[: rot // 2] = (np.float32(1.0) / np.power(np.float64(np.float32(theta)), ex.astype(np.float64)).astype(np.float32))
    return f


def rope_float(x: np.ndarray, pos: np.ndarray, inv: np.ndarray) -> np.ndarray:
    """x [..., T, H, dh] float32 with positions pos [..., T]: the reference's float32 rotation."""
    half = x.shape[-1] // 2
    ang = pos.astype(np.float32)[..., None] * inv[None, :]  # float32 product
    c = np.cos(ang.astype(np.float64)).astype(np.float32)[..., None, :]
    s = np.sin(ang.astype(np.float64)).astype(np.float32)[..., None, :]
    a, b = x[..., :half], x[..., half:]
    lo = a * c + (-b) * s
    hi = b * c + a * s
    return np.concatenate([lo, hi], axis=-1).astype(np.float32)


def _softmax_apply(scores: np.ndarray, allowed: np.ndarray, v: np.ndarray) -> np.ndarray:
    """scores [..., Q, K] float64, allowed bool broadcastable, v [..., K, dh] -> [..., Q, dh]; zeros if none."""
    s = np.where(allowed, scores, -np.inf)
    m = np.max(s, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.where(allowed, np.exp(s - m), 0.0)
    z = p.sum(axis=-1, keepdims=True)
    o = p @ v
    return np.where(z > 0, o / np.where(z > 0, z, 1.0), 0.0)


def split_qkv(qkv: np.ndarray, rows: int, n: int, heads: int, dh: int, inner: int):
    x = qkv.reshape(rows, n, 3 * inner)
    q = x[:, :, 0 : heads * dh].reshape(rows, n, heads, dh)
    k = x[:, :, inner : inner + heads * dh].reshape(rows, n, heads, dh)
    v = x[:, :, 2 * inner : 2 * inner + heads * dh].reshape(rows, n, heads, dh)
    return q, k, v


def c2_time(qkv, live, rows, n, heads, dh, inner, theta=10000.0):
    q, k, v = split_qkv(np.asarray(qkv, np.float32), rows, n, heads, dh, inner)
    pos = np.broadcast_to(np.arange(n), (rows, n))
    inv = inv_freq(dh, theta)
    qr = rope_float(q, pos, inv).astype(np.float64).transpose(0, 2, 1, 3)  # r h t e
    kr = rope_float(k, pos, inv).astype(np.float64).transpose(0, 2, 1, 3)
    vv = v.astype(np.float64).transpose(0, 2, 1, 3)
    s = qr @ kr.transpose(0, 1, 3, 2)  # r h q k
    allowed = np.asarray(live, bool).reshape(rows, 1, 1, n)
    o = _softmax_apply(s, allowed, vv)  # r h q e
    out = np.zeros((rows, n, inner), np.float64)
    out[:, :, : heads * dh] = o.transpose(0, 2, 1, 3).reshape(rows, n, heads * dh)
    return out.reshape(rows * n, inner).astype(np.float32)


def c2_group(qkv, live, group, rows, n, heads, dh, inner):
    q, k, v = split_qkv(np.asarray(qkv, np.float32), rows, n, heads, dh, inner)
    q = q.astype(np.float64).transpose(1, 2, 0, 3)  # t h r e
    k = k.astype(np.float64).transpose(1, 2, 0, 3)
    v = v.astype(np.float64).transpose(1, 2, 0, 3)
    g = np.asarray(group)
    same = g[:, None] == g[None, :]  # q-row x k-row
    lv = np.asarray(live, bool).reshape(rows, n).T  # t x k-row
    allowed = same[None, None, :, :] & lv[:, None, None, :]
    s = q @ k.transpose(0, 1, 3, 2)
    o = _softmax_apply(s, allowed, v)  # t h r e
    out = np.zeros((rows, n, inner), np.float64)
    out[:, :, : heads * dh] = o.transpose(2, 0, 1, 3).reshape(rows, n, heads * dh)
    return out.reshape(rows * n, inner).astype(np.float32)


def ts_time_allowed(key_valid, known, rows, enc, ll, n) -> np.ndarray:
    """[rows, n(q), n(k)] from BlockLayout.timeAllowed's rules, enumerated independently."""
    kv = np.asarray(key_valid, bool).reshape(rows, enc)
    kn = np.asarray(known, bool).reshape(rows)
    qi = np.arange(n)[:, None]
    ki = np.arange(n)[None, :]
    valid = np.zeros((rows, n), bool)
    valid[:, :enc] = kv
    enc_q = qi < enc
    enc_k = ki < enc
    a_enc = enc_k[None] & ((ki == qi)[None] | (valid[:, None, :] & ((ki <= qi)[None] | kn[:, None, None])))
    a_dec = np.where(enc_k[None], (ki < ll)[None] & valid[:, None, :], (ki <= qi)[None])
    return np.where(enc_q[None], a_enc, a_dec)


def ts_time(qkv, key_valid, known, pos, rows, enc, ll, n, heads, dh, d, rope_dim, theta=10000.0):
    q, k, v = split_qkv(np.asarray(qkv, np.float32), rows, n, heads, dh, d)
    inv = inv_freq(dh, theta, rope_dim)
    p = np.asarray(pos).reshape(rows, n)
    qr = rope_float(q, p, inv).astype(np.float64).transpose(0, 2, 1, 3)
    kr = rope_float(k, p, inv).astype(np.float64).transpose(0, 2, 1, 3)
    vv = v.astype(np.float64).transpose(0, 2, 1, 3)
    s = (qr @ kr.transpose(0, 1, 3, 2)) * (1.0 / np.sqrt(dh))
    allowed = ts_time_allowed(key_valid, known, rows, enc, ll, n)[:, None]
    o = _softmax_apply(s, allowed, vv)
    out = np.zeros((rows, n, d), np.float64)
    out[:, :, : heads * dh] = o.transpose(0, 2, 1, 3).reshape(rows, n, heads * dh)
    return out.reshape(rows * n, d).astype(np.float32)


def ts_variate_allowed(key_valid, group, role, covariates, rows, enc, n) -> np.ndarray:
    """[n(slot), rows(q), rows(k)] from BlockLayout.variateAllowed's rules."""
    g = np.asarray(group)
    rl = np.asarray(role)
    kv = np.asarray(key_valid, bool).reshape(rows, enc)
    same = g[:, None] == g[None, :]
    eye = np.eye(rows, dtype=bool)
    if covariates:
        forbid = ((rl[:, None] != 0) & (rl[None, :] == 0)) | ((rl[:, None] == 2) & (rl[None, :] != 2))
    else:
        forbid = np.zeros((rows, rows), bool)
    out = np.zeros((n, rows, rows), bool)
    for t in range(n):
        valid_k = kv[:, t] if t < enc else np.ones(rows, bool)
        out[t] = same & (eye | (valid_k[None, :] & ~forbid))
    return out


def ts_variate(qkv, key_valid, group, role, covariates, rows, enc, n, heads, dh, d):
    q, k, v = split_qkv(np.asarray(qkv, np.float32), rows, n, heads, dh, d)
    q = q.astype(np.float64).transpose(1, 2, 0, 3)
    k = k.astype(np.float64).transpose(1, 2, 0, 3)
    v = v.astype(np.float64).transpose(1, 2, 0, 3)
    allowed = ts_variate_allowed(key_valid, group, role, covariates, rows, enc, n)[:, None]
    s = (q @ k.transpose(0, 1, 3, 2)) * (1.0 / np.sqrt(dh))
    o = _softmax_apply(s, allowed, v)
    out = np.zeros((rows, n, d), np.float64)
    out[:, :, : heads * dh] = o.transpose(2, 0, 1, 3).reshape(rows, n, heads * dh)
    return out.reshape(rows * n, d).astype(np.float32)
