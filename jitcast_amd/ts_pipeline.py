"""Timestral's forecasting pipeline on the host: TimestralPipeline.forecast around any block forward
(J/timestral/TimestralPipeline.java:39-523), with the pieces it calls.

  split_windows        SeriesWindows.split (J/host/SeriesWindows.java:36-56): consecutive series, at most
                       batch_size of them and max_tokens tokens, at least one series per window
  sign_complement, sign_average
                       SignFlip.complement / average (J/host/SignFlip.java:52-79)
  target_encode        TargetEncoding.apply (J/timestral/TargetEncoding.java:38-167): categorical
                       covariates become the smoothed mean of the target where each code occurs
  last_loc_scale, advancing_frames, clamp_non_finite
                       Scaler.lastLocScale / advancingFrames / clampNonFinite
                       (J/timestral/Scaler.java:66-84, 143-236), in double where the reference is
  TimestralPipeline    windows, batch assembly (one row per target and covariate, right-aligned,
                       capped at max_context, left-padded to whole patches), block-autoregressive
                       decoding with each block moved to the advancing refine frame and its median fed
                       back, the cap to the observed range, sign-flip averaging and the non-negative
                       clip (TimestralPipeline.java:165-523)

The forward is any callable forward(inputs, observed, group, h, role, known_future, known_future_mask)
returning [rows][h * patch][quantiles] float32, as BlockForward.predictBlock (HipTimestralModel's
predict_block). Every float operation rounds as the reference's float / double code does: sums that
the reference runs in order run in order here, across rows at once.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, replace

import numpy as np

from . import _lib
from . import options as opts
from .api import Forecast, TimeSeries

f32 = np.float32
DEFAULT_BATCH_SIZE = 512
TARGET, PAST, KNOWN = 0, 1, 2  # BlockInput roles
_F32_MAX = float(np.finfo(np.float32).max)


def default_max_tokens() -> int:
    """-Dtimestral.maxTokens, default 131,072 (TimestralPipeline.defaultMaxTokens)."""
    return opts.number("timestral.maxTokens", 131_072, 1)


# ---- SeriesWindows, SignFlip -------------------------------------------------------------------

def split_windows(series: list, batch_size: int, max_tokens: int, patches: int) -> list:
    """[start, end) windows of consecutive series: at most batch_size series and max_tokens tokens
    (patches per row), but always at least one series."""
    out, n, start = [], len(series), 0
    while start < n:
        end, tokens = start, 0
        while end < n and end - start < batch_size:
            t = series[end].rows() * patches
            if end > start and tokens + t > max_tokens:
                break
            tokens += t
            end += 1
        out.append((start, end))
        start = end
    return out


def sign_complement(levels) -> np.ndarray:
    """complement[i] = the level closest to 1 - q[i] (float32 arithmetic, the first on ties); a
    quantile set not symmetric within 1e-6 is rejected."""
    q = np.asarray(levels, np.float32)
    c = np.empty(q.size, np.int64)
    for i in range(q.size):
        target = f32(f32(1) - q[i])
        d = np.abs(q - target)
        best = int(np.argmin(d))  # argmin keeps the first of equal distances, as the strict < scan
        if float(d[best]) > 1e-6:
            raise RuntimeError("sign-flip TTA needs a symmetric quantile set")
        c[i] = best
    return c


def sign_average(a: np.ndarray, b: np.ndarray, complement: np.ndarray, h: int) -> None:
    """a[t][q][:h] = (a[t][q][:h] + -b[t][complement[q]][:h]) / 2 in place (float32)."""
    a[:, :, :h] = (a[:, :, :h] + -b[:, complement, :h]) / f32(2)


# ---- TargetEncoding ----------------------------------------------------------------------------

_SMOOTH = 1.0


def _encoding_target(row: np.ndarray, max_context: int) -> np.ndarray:
    """_encoding_target: the forward-filled target from its first observation on, within the last
    max_context steps, NaN elsewhere (double)."""
    t = row.size
    obs = np.isfinite(row)
    idx = np.where(obs, np.arange(t), -1)
    last = np.maximum.accumulate(idx)
    out = np.where(last >= 0, row.astype(np.float64)[np.maximum(last, 0)], np.nan)
    out[: max(t - max_context, 0)] = np.nan
    return out


def _code_key(v: float):
    """Double.compare's order for finite codes: -0.0 before 0.0 (distinct categories)."""
    return (v, 0 if math.copysign(1.0, v) < 0 else 1)


def _encode(target: np.ndarray, past: np.ndarray, future):
    """target_encode: ({past}, {future} or None) as float32."""
    fin = np.isfinite(target)
    count = float(np.count_nonzero(fin))
    s = 0.0
    for v in target[fin]:  # in order, as the reference sums
        s += float(v)
    mean = s / count if count > 0 else 0.0
    cats = sorted({_code_key(float(v)) for v in past if math.isfinite(v)})
    index = {k: i for i, k in enumerate(cats)}
    nan_slot = len(cats)

    def slot(code: float) -> int:
        if math.isnan(code):
            return nan_slot
        return index.get(_code_key(code), -1)

    sums = [0.0] * (nan_slot + 1)
    counts = [0.0] * (nan_slot + 1)
    slots = []
    for i in range(target.size):
        sl = slot(float(past[i]))
        if sl < 0:
            raise RuntimeError("every past code must be a category")
        slots.append(sl)
        if fin[i]:
            sums[sl] += float(target[i])
            counts[sl] += 1.0
    lookup = [(_SMOOTH * mean + sums[k]) / (_SMOOTH + counts[k]) for k in range(nan_slot + 1)] + [mean]
    enc_past = np.asarray([lookup[k] for k in slots], np.float64).astype(np.float32)
    if future is None:
        return enc_past, None
    enc_future = np.asarray([lookup[slot(float(c)) if slot(float(c)) >= 0 else nan_slot + 1] for c in future],
                            np.float64).astype(np.float32)
    return enc_past, enc_future


def _encode_row(target, codes: np.ndarray, length: int, horizon: int) -> np.ndarray:
    if target is None:
        return codes[: length + horizon].astype(np.float32)
    past = codes[:length]
    future = codes[length:length + horizon] if horizon > 0 else None
    enc_p, enc_f = _encode(target, past, future)
    out = np.empty(length + horizon, np.float32)
    # a missing code before the target starts is padding, not the missing category
    out[:length] = np.where(np.isnan(target) & np.isnan(past), np.float32(np.nan), enc_p)
    if enc_f is not None:
        out[length:] = enc_f
    return out


def target_encode(ts: TimeSeries, horizon: int, max_context: int) -> TimeSeries:
    """The series with its categorical covariates encoded and appended after its numeric ones
    (past rows after the numeric past covariates, known rows after the numeric future ones)."""
    if not ts.has_categorical():
        return ts
    length = ts.length()
    target = _encoding_target(ts.target[0], max_context) if ts.targets() == 1 else None
    past = [_encode_row(target, c, length, 0) for c in (ts.past_categorical or ())]
    known = []
    for c in ts.future_categorical or ():
        if c.size < length + horizon:
            raise ValueError(f"future categorical covariates need at least {length + horizon} steps, got {c.size}")
        known.append(_encode_row(target, c, length, horizon))
    cat = lambda a, b: (list(a or ()) + b) or None  # noqa: E731
    return TimeSeries(list(ts.target), cat(ts.past_covariates, past), cat(ts.future_covariates, known))


# ---- Scaler ------------------------------------------------------------------------------------

def context_stats(x: np.ndarray, observed: np.ndarray, minimum_scale: float):
    """(loc, scale, lo, hi) float32 [rows] of each row (jc_ts_context_stats): Scaler.lastLocScale's
    causal mean and Bessel-corrected std of every observed value (a running sum in double, in order)
    and the smallest and largest observed value (0 when none is)."""
    x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
    m = np.ascontiguousarray(np.atleast_2d(observed), np.uint8)
    rows, t = x.shape
    if m.shape != x.shape:
        raise ValueError(f"observed {m.shape} does not match the values {x.shape}")
    out = [np.empty(rows, np.float32) for _ in range(4)]
    _lib.call("jc_ts_context_stats", x.ctypes.data, m.ctypes.data, rows, t, ctypes.c_float(minimum_scale),
              *(o.ctypes.data for o in out))
    return tuple(out)


def last_loc_scale(x: np.ndarray, observed: np.ndarray, minimum_scale: float):
    """(loc, scale) float32 [rows] of each row's last patch: Scaler.lastLocScale
    (Scaler.java:65-79), the causal mean and Bessel-corrected std of every observed value."""
    loc, scale, _, _ = context_stats(x, observed, minimum_scale)
    return loc, scale


def advancing_frames(context: np.ndarray, observed: np.ndarray, sinh_median: np.ndarray, patch: int,
                     minimum_scale: float):
    """(loc, scale) double [rows, H] of each decoded patch in the advancing refine frame
    (jc_ts_advancing_frames, Scaler.advancingFrames): patch j uses the statistics of the observed
    context plus the block's medians of patches 0..j-1, each folded in after being denormalised in
    its own frame. context / observed [rows, T] (T a multiple of the patch), sinh_median
    [rows, H, patch] (median - loc) / scale of the last context patch."""
    ctx = np.ascontiguousarray(context, np.float32)
    m = np.ascontiguousarray(observed, np.uint8)
    sm = np.ascontiguousarray(sinh_median, np.float64)
    rows, t = ctx.shape
    n_pred = sm.shape[1]
    if m.shape != ctx.shape or sm.shape != (rows, n_pred, patch):
        raise ValueError(f"shapes disagree: context {ctx.shape}, observed {m.shape}, sinh_median {sm.shape}")
    locs = np.empty((rows, n_pred))
    scales = np.empty((rows, n_pred))
    _lib.call("jc_ts_advancing_frames", ctx.ctypes.data, m.ctypes.data, sm.ctypes.data, rows, t, patch, n_pred,
              ctypes.c_float(minimum_scale), locs.ctypes.data, scales.ctypes.data)
    return locs, scales


def clamp_non_finite(v: np.ndarray) -> np.ndarray:
    """Along the last axis: +-inf to the largest / smallest finite value, a vector with no finite
    value to 0; NaN kept."""
    fin = np.isfinite(v)
    mx = np.where(fin, v, -np.inf).max(axis=-1, keepdims=True)
    mn = np.where(fin, v, np.inf).min(axis=-1, keepdims=True)
    x = np.where(v == np.inf, mx, np.where(v == -np.inf, mn, v))
    return np.where(np.isinf(x), f32(0), x).astype(np.float32)


# ---- the pipeline ------------------------------------------------------------------------------

@dataclass(frozen=True)
class Options:
    """TimestralPipeline.Options: context cap in steps, patches decoded per block, the cap factor k
    (0 disables), the fed-back median's magnitude limit, sign-flip averaging, non-negative clip."""

    max_context: int
    per_shot_horizon_patches: int
    cap_k: float
    extreme_value_threshold: float
    symmetric_averaging: bool
    clip_nonnegative: bool

    @staticmethod
    def defaults(c) -> "Options":
        return Options(c.context_length, 32, float(f32(1e4)), float(f32(1e30)), True, True)

    def with_symmetric_averaging(self, on: bool) -> "Options":
        return replace(self, symmetric_averaging=bool(on))

    def with_clip_nonnegative(self, on: bool) -> "Options":
        return replace(self, clip_nonnegative=bool(on))


@dataclass
class Assembled:
    rows: np.ndarray          # float32 [R, padded]
    mask: np.ndarray          # bool [R, padded]
    group: np.ndarray         # int32 [R]: the series' index in the window
    role: np.ndarray | None   # int32 [R] when any series has covariates
    known_future: np.ndarray | None       # float32 [R, ceil(H/P)*P] when any series has known ones
    known_future_mask: np.ndarray | None  # bool, same shape
    target_rows: list         # per series: its target rows' indices


def non_negative(row: np.ndarray) -> bool:
    """Whether every finite value is >= 0 and one exists."""
    fin = row[np.isfinite(row)]
    return fin.size > 0 and not bool((fin < 0).any())


def forward_fill(x: np.ndarray, m: np.ndarray) -> np.ndarray:
    """ffill_with_mask: unobserved positions take the last observed value; leading ones take x[0]."""
    if m.all():  # nothing to fill
        return np.asarray(x, np.float32)
    idx = np.where(m, np.arange(x.size), -1)
    last = np.maximum.accumulate(idx)
    return np.where(m, x, np.where(last >= 0, x[np.maximum(last, 0)], x[0])).astype(np.float32)


def _neg_clip(x: np.ndarray) -> np.ndarray:
    """Math.max(x, 0f) element-wise: -0.0 and negatives to +0.0, NaN kept."""
    return np.where((x < 0) | ((x == 0) & np.signbit(x)), f32(0), x).astype(np.float32)


class TimestralPipeline:
    """TimestralPipeline: forecast(series, horizon) around a block forward."""

    def __init__(self, config, forward, options: Options | None = None, batch_size: int = DEFAULT_BATCH_SIZE,
                 max_tokens: int | None = None):
        options = Options.defaults(config) if options is None else options
        max_tokens = default_max_tokens() if max_tokens is None else max_tokens
        if batch_size < 1 or max_tokens < 1:
            raise ValueError("batchSize and maxTokens must be >= 1")
        if options.max_context < config.patch_size or options.per_shot_horizon_patches < 1:
            raise ValueError("maxContext must hold a patch and perShotHorizonPatches must be >= 1")
        self.config, self.forward, self._options = config, forward, options
        self.batch_size, self.max_tokens = batch_size, max_tokens
        self._complement = sign_complement(config.quantiles) if options.symmetric_averaging else None

    def options(self) -> Options:
        return self._options

    def with_options(self, o: Options) -> "TimestralPipeline":
        return TimestralPipeline(self.config, self.forward, o, self.batch_size, self.max_tokens)

    def with_max_tokens(self, tokens: int) -> "TimestralPipeline":
        return TimestralPipeline(self.config, self.forward, self._options, self.batch_size, tokens)

    def forecast(self, series: list, horizon: int) -> list:
        """One Forecast per series, in order (ForecastEngine.forecast)."""
        if horizon < 1:
            raise ValueError(f"horizon must be >= 1, got {horizon}")
        c, o = self.config, self._options
        ps = c.patch_size
        max_len = max((ts.length() for ts in series), default=0)
        per_shot = min(o.per_shot_horizon_patches, c.block_size)
        patches = (min(max_len, o.max_context) + ps - 1) // ps + 2 * min(per_shot, (horizon + ps - 1) // ps)
        out = []
        for a, b in split_windows(series, self.batch_size, self.max_tokens, patches):
            out.extend(self._forecast_window(series[a:b], horizon))
        return out

    def _forecast_window(self, series: list, horizon: int) -> list:
        c, o = self.config, self._options
        for ts in series:
            if ts.rows() > ts.targets() and not c.covariate_enabled:
                raise ValueError("this checkpoint was not trained with covariates")
            if ts.future_count() + ts.future_categorical_count() > 0 and not c.supports_known_covariates():
                raise ValueError("this checkpoint cannot condition on known-future covariates")
        encoded = [target_encode(ts, horizon, o.max_context) for ts in series]
        a = self._forecast_raw(encoded, horizon, 1.0)
        if o.symmetric_averaging:
            b = self._forecast_raw(encoded, horizon, -1.0)
            for s in range(len(a)):
                sign_average(a[s], b[s], self._complement, horizon)
        levels = np.asarray(c.quantiles, np.float32)
        out = []
        for s, ts in enumerate(series):
            f = a[s]
            if o.clip_nonnegative:
                for v in range(f.shape[0]):
                    if non_negative(ts.target[v]):
                        f[v] = _neg_clip(f[v])
            out.append(Forecast(levels, f))
        return out

    def assemble(self, series: list, horizon: int, sign: float) -> Assembled:
        """_assemble_rows for a window, every value multiplied by sign."""
        c, o = self.config, self._options
        ps = c.patch_size
        sg = f32(sign)
        t = max((ts.length() for ts in series), default=0)
        hlen = (horizon + ps - 1) // ps * ps
        covariates = any(ts.past_count() > 0 or ts.future_count() > 0 for ts in series)
        any_known = any(ts.future_count() > 0 for ts in series)
        rows, masks, groups, roles, kf, kfm, target_rows = [], [], [], [], [], [], []

        def add_cov(values, length, role, future):
            x = np.zeros(t, np.float32)
            m = np.zeros(t, bool)
            v = values[:length]
            obs = ~np.isnan(v)
            m[t - length:] = obs
            x[t - length:] = np.where(obs, sg * v, f32(0))
            rows.append(x)
            masks.append(m)
            groups.append(s)
            roles.append(role)
            fv = np.zeros(hlen, np.float32)
            fm = np.zeros(hlen, bool)
            if future is not None:
                fut = future[length:length + horizon]
                fm[:horizon] = ~np.isnan(fut)
                fv[:horizon] = np.where(fm[:horizon], sg * fut, f32(0))
            kf.append(fv)
            kfm.append(fm)

        for s, ts in enumerate(series):
            length = ts.length()
            tr = []
            for v in range(ts.targets()):
                tr.append(len(rows))
                val = ts.target[v]
                x = np.zeros(t, np.float32)
                m = np.zeros(t, bool)
                obs = np.isfinite(val)
                m[t - length:] = obs
                # missing targets are zeroed, then negated: -0.0 in the mirrored pass
                x[t - length:] = sg * np.where(obs, val, f32(0))
                rows.append(forward_fill(x, m))
                masks.append(m)
                groups.append(s)
                roles.append(TARGET)
                kf.append(np.zeros(hlen, np.float32))
                kfm.append(np.zeros(hlen, bool))
            target_rows.append(tr)
            for v in range(ts.past_count()):
                add_cov(ts.past_covariates[v], length, PAST, None)
            for v in range(ts.future_count()):
                fc = ts.future_covariates[v]
                if fc.size < length + horizon:
                    raise ValueError(f"future covariates of series {s} need at least {length + horizon} steps, "
                                     f"got {fc.size}")
                add_cov(fc, length, KNOWN, fc)
        kept = min(t, o.max_context)
        padded = (kept + ps - 1) // ps * ps
        r = np.zeros((len(rows), padded), np.float32)
        m = np.zeros((len(rows), padded), bool)
        if rows:
            r[:, padded - kept:] = np.stack(rows)[:, t - kept:]
            m[:, padded - kept:] = np.stack(masks)[:, t - kept:]
        return Assembled(r, m, np.asarray(groups, np.int32), np.asarray(roles, np.int32) if covariates else None,
                         np.stack(kf) if any_known else None, np.stack(kfm) if any_known else None, target_rows)

    def _forecast_raw(self, series: list, horizon: int, sign: float) -> list:
        """One forecast pass: per series float32 [targets][quantiles][horizon]."""
        c = self.config
        a = self.assemble(series, horizon, sign)
        q = self._decode(a, horizon)
        bounds = self._cap_bounds(a.rows, a.mask)
        out = []
        for s in range(len(series)):
            tr = a.target_rows[s]
            f = np.transpose(q[tr], (0, 2, 1)).copy()  # [targets][Q][horizon]
            if bounds is not None:
                lo, hi = bounds[0][tr][:, None, None], bounds[1][tr][:, None, None]
                f = np.minimum(np.maximum(f, lo), hi)  # Math.min(Math.max(x, b0), b1): NaN kept
            if np.isnan(f).any():
                raise RuntimeError("forecast produced NaN values: the input is degenerate, or an activation left "
                                   "the FP32 range")
            out.append(f.astype(np.float32))
        return out

    def _cap_bounds(self, rows: np.ndarray, mask: np.ndarray):
        """_cap_quantiles (TimestralPipeline.java:378-395): [min - k s, max + k s] of each row's observed
        context (float32), or None."""
        o = self._options
        if o.cap_k <= 0:
            return None
        _, scale, mn, mx = context_stats(rows, mask, self.config.minimum_scale)
        s = scale * f32(o.cap_k)
        return (mn - s).astype(np.float32), (mx + s).astype(np.float32)

    def _decode(self, a: Assembled, horizon: int) -> np.ndarray:
        """_block_ar_decode: [rows][horizon][quantiles], block after block, the context growing by each
        block's feedback (targets their median, known covariates their future, past a blank)."""
        c, o = self.config, self._options
        ps = c.patch_size
        r = a.rows.shape[0]
        per_shot = min(o.per_shot_horizon_patches, c.block_size)
        med = c.median_index
        context, mask = a.rows, a.mask
        out = np.zeros((r, horizon, c.num_quantiles), np.float32)
        remaining = (horizon + ps - 1) // ps
        offset = 0
        role = a.role if a.role is not None else np.full(r, TARGET, np.int32)
        while remaining > 0:
            block = min(per_shot, remaining)
            blen = block * ps
            kf = None if a.known_future is None else np.ascontiguousarray(a.known_future[:, offset:offset + blen])
            kfm = None if a.known_future_mask is None else np.ascontiguousarray(a.known_future_mask[:, offset:offset + blen])
            q = np.asarray(self.forward(context, mask, a.group, block, a.role, kf, kfm), np.float32).copy()
            self._refine(q, context, mask, a.role)
            n = min(blen, horizon - offset)
            out[:, offset:offset + n] = q[:, :n]
            remaining -= block
            offset += blen
            if remaining <= 0:
                break
            length = context.shape[1] + blen
            keep = max(ps, o.max_context // ps * ps) if length > o.max_context else length
            med_v = q[:, :, med]
            fb = np.where(np.isfinite(med_v) & (np.abs(med_v) < f32(o.extreme_value_threshold)), med_v, f32(0))
            fm = np.ones((r, blen), bool)
            if a.role is not None:
                if kf is not None:  # known covariates take their real future
                    known = (role == KNOWN)[:, None]
                    fb = np.where(known, kf, fb)
                    fm = np.where(known, kfm, fm)
                past = (role == PAST)[:, None]  # past-only covariates a blank
                fb = np.where(past, f32(0), fb)
                fm = np.where(past, False, fm)
            row = np.concatenate([context, fb.astype(np.float32)], axis=1)
            m = np.concatenate([mask, fm], axis=1)
            context = np.ascontiguousarray(row[:, length - keep:])
            mask = np.ascontiguousarray(m[:, length - keep:])
        return out

    def _refine(self, q: np.ndarray, context: np.ndarray, mask: np.ndarray, role) -> None:
        """_refine_block, in place: a decoded block of the target rows moved from the frame of the last
        context patch to the advancing refine frame; the first horizon patch keeps its frame."""
        c = self.config
        ps = c.patch_size
        n_pred = q.shape[1] // ps
        if n_pred <= 1:
            return
        sel = np.arange(q.shape[0]) if role is None else np.nonzero(np.asarray(role) == TARGET)[0]
        if sel.size == 0:
            return
        ctx, msk = context[sel], mask[sel]
        loc0, scale0 = last_loc_scale(ctx, msk, c.minimum_scale)
        med = q[sel][:, :, c.median_index].reshape(sel.size, n_pred, ps).astype(np.float64)
        sinh_median = (med - loc0.astype(np.float64)[:, None, None]) / scale0.astype(np.float64)[:, None, None]
        locs, scales = advancing_frames(ctx, msk, sinh_median, ps, c.minimum_scale)
        lj = locs.astype(np.float32)
        sj = scales.astype(np.float32)
        lj[:, 0] = loc0
        sj[:, 0] = scale0
        blk = q[sel].reshape(sel.size, n_pred, ps, -1)
        v = (blk - loc0[:, None, None, None]) / scale0[:, None, None, None] * sj[:, :, None, None] + lj[:, :, None, None]
        q[sel] = clamp_non_finite(v.astype(np.float32)).reshape(sel.size, n_pred * ps, -1)
