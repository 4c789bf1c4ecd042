"""Chronos-2's quantile helpers for the long-horizon unrolling (J/chronos2/QuantileMath.java:24-150):
the probability mass of each level, linear interpolation between levels, and the quantiles of a
weighted sample. Every operation rounds as the reference does: float32 arithmetic with no fused
multiply-add, the cumulative weights summed in double, sorts stable in Float.compare's order
(-0.0 before 0.0, NaN after +inf). Rows are processed together (numpy) rather than one by one.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
F32_MAX = np.float32(np.finfo(np.float32).max)


def probability_mass(levels) -> np.ndarray:
    """QuantileMath.probabilityMass (QuantileMath.java:32-47): (q[i+1] - q[i-1]) / 2 with q[-1] = 0
    and q[n] = 1, each divided by their float sum (summed in order)."""
    lv = np.asarray(levels, F32)
    b = np.concatenate([[F32(0)], lv, [F32(1)]]).astype(F32)
    m = ((b[2:] - b[:-2]) / F32(2)).astype(F32)
    total = F32(0)
    for v in m:  # sequential float adds, as the reference's loop
        total = F32(total + v)
    return (m / total).astype(F32)


def float_compare_key(v: np.ndarray) -> np.ndarray:
    """int64 keys whose order is Float.compare's: the IEEE bits with negative values flipped, every
    NaN the canonical NaN (above +inf), -0.0 below 0.0."""
    v = np.ascontiguousarray(v, F32)
    bits = v.view(np.int32).astype(np.int64)
    bits = np.where(np.isnan(v), np.int64(0x7FC00000), bits)
    return np.where(bits < 0, -(bits & 0x7FFFFFFF) - 1, bits)


def _nan_to_num(v: np.ndarray) -> np.ndarray:
    """torch.nan_to_num: NaN to 0, +-inf to the largest finite floats."""
    return np.nan_to_num(v, nan=0.0, posinf=F32_MAX, neginf=-F32_MAX).astype(F32)


def interpolate(query, levels, values) -> np.ndarray:
    """QuantileMath.interpolate (QuantileMath.java:49-100): each row's values at the query levels from
    its values at its own levels (levels [rows, n] or one [n] row shared by all), sorted by level;
    the end values extend to 0 and 1 when the batch's smallest level is above 0 / largest below 1
    (decided once for the whole batch). Returns float32 [rows, len(query)]."""
    q = np.asarray(query, F32)
    vals = np.asarray(values, F32)
    rows, n = vals.shape
    lv = np.asarray(levels, F32)
    if lv.ndim == 1:
        lv = np.broadcast_to(lv, (rows, n))
    if rows == 0:
        return np.zeros((0, q.size), F32)
    pad_low = bool(lv.min() > 0)
    pad_high = bool(lv.max() < 1)
    order = np.argsort(float_compare_key(lv), axis=1, kind="stable")
    sl = np.take_along_axis(lv, order, axis=1)
    sv = np.take_along_axis(vals, order, axis=1)
    if pad_low:
        sl = np.concatenate([np.zeros((rows, 1), F32), sl], axis=1)
        sv = np.concatenate([sv[:, :1], sv], axis=1)
    if pad_high:
        sl = np.concatenate([sl, np.ones((rows, 1), F32)], axis=1)
        sv = np.concatenate([sv, sv[:, -1:]], axis=1)
    m = sl.shape[1]
    out = np.empty((rows, q.size), F32)
    ridx = np.arange(rows)
    for j, qj in enumerate(q):
        # torch.searchsorted(right=True): the first level above q (the levels are ascending)
        upper = np.minimum((sl <= qj).sum(axis=1), m - 1)
        lower = np.maximum(upper - 1, 0)
        lo_l, up_l = sl[ridx, lower], sl[ridx, upper]
        lo_v, up_v = sv[ridx, lower], sv[ridx, upper]
        with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
            w = _nan_to_num(((qj - lo_l).astype(F32) / (up_l - lo_l).astype(F32)).astype(F32))
            out[:, j] = (lo_v + (w * (up_v - lo_v).astype(F32)).astype(F32)).astype(F32)
    return out


def weighted_quantile(query, weights, samples) -> np.ndarray:
    """QuantileMath.weightedQuantile (QuantileMath.java:102-136): per row, the samples sorted, their
    normalized weights accumulated in double into levels (rounded to float, clamped to [0, 1]), and
    the query levels interpolated. weights [n]; samples [rows, n]."""
    w = np.asarray(weights, F32)
    s = np.asarray(samples, F32)
    total = F32(0)
    for v in w:
        total = F32(total + v)
    norm = (w / total).astype(F32)
    order = np.argsort(float_compare_key(s), axis=1, kind="stable")
    srt = np.take_along_axis(s, order, axis=1)
    cum = np.cumsum(norm[order].astype(np.float64), axis=1)  # sequential double adds per row
    lv = np.clip(cum.astype(F32), F32(0), F32(1)).astype(F32)
    return interpolate(query, lv, srt)
