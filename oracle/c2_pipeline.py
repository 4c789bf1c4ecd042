"""A scalar restatement of Chronos-2's host pipeline and its quantile helpers, loop by loop as the
reference writes them, with float32 scalars for every float operation.

TEST INFRASTRUCTURE ONLY: the checker for jitcast_amd.pipeline and jitcast_amd.quantile_math, which
compute the same things with array operations. Nothing here imports the product.

  probability_mass, interpolate, weighted_quantile   J/chronos2/QuantileMath.java:32-136
  forecast                                          J/chronos2/Chronos2Pipeline.java:190-448: every
      forward call's arguments go through `forward(context, group, future, output_patches)`, which
      returns [rows][Q][output_patches * P]; the result is per series [targets][Q][horizon]
"""
from __future__ import annotations

import math

import numpy as np

f32 = np.float32
F32_MAX = f32(np.finfo(np.float32).max)


def _fc_key(v):
    """Float.compare's order as a Python sort key: numbers ascending, -0.0 before 0.0, NaN last."""
    v = float(v)
    if math.isnan(v):
        return (2, 0.0, 0)
    return (1, v, 0 if math.copysign(1.0, v) < 0 else 1)


def probability_mass(levels):
    """QuantileMath.probabilityMass (QuantileMath.java:32-47)."""
    n = len(levels)
    b = [f32(0)] + [f32(x) for x in levels] + [f32(1)]
    m = []
    total = f32(0)
    for i in range(n):
        m.append(f32(f32(b[i + 2] - b[i]) / f32(2)))
        total = f32(total + m[i])
    return [f32(x / total) for x in m]


def _nan_to_num(v):
    if math.isnan(v):
        return f32(0)
    if v == math.inf:
        return F32_MAX
    if v == -math.inf:
        return -F32_MAX
    return f32(v)


def interpolate(query, levels, values):
    """QuantileMath.interpolate (QuantileMath.java:49-100): levels[r], values[r] per row."""
    rows = len(values)
    lo_all, hi_all = math.inf, -math.inf
    for lv in levels:
        for v in lv:
            lo_all = min(lo_all, float(v))
            hi_all = max(hi_all, float(v))
    pad_low, pad_high = lo_all > 0, hi_all < 1
    out = []
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        for r in range(rows):
            lr = [f32(x) for x in levels[r]]
            n = len(lr)
            order = sorted(range(n), key=lambda i: _fc_key(lr[i]))
            sl, sv = [], []
            if pad_low:
                sl.append(f32(0))
                sv.append(f32(values[r][order[0]]))
            for i in range(n):
                sl.append(lr[order[i]])
                sv.append(f32(values[r][order[i]]))
            if pad_high:
                sl.append(f32(1))
                sv.append(f32(values[r][order[n - 1]]))
            m = len(sl)
            row = []
            for q in query:
                q = f32(q)
                upper = 0
                while upper < m and sl[upper] <= q:
                    upper += 1
                upper = min(upper, m - 1)
                lower = max(upper - 1, 0)
                w = _nan_to_num(f32(f32(q - sl[lower]) / f32(sl[upper] - sl[lower])))
                row.append(f32(sv[lower] + f32(w * f32(sv[upper] - sv[lower]))))
            out.append(row)
    return out


def weighted_quantile(query, weights, samples):
    """QuantileMath.weightedQuantile (QuantileMath.java:102-136)."""
    n = len(weights)
    total = f32(0)
    for w in weights:
        total = f32(total + f32(w))
    norm = [f32(f32(w) / total) for w in weights]
    levels, srt = [], []
    for s in samples:
        order = sorted(range(n), key=lambda i: _fc_key(s[i]))
        acc = 0.0
        lv, sv = [], []
        for i in range(n):
            sv.append(f32(s[order[i]]))
            acc += float(norm[order[i]])
            lv.append(min(max(f32(acc), f32(0)), f32(1)))
        levels.append(lv)
        srt.append(sv)
    return interpolate(query, levels, srt)


def forecast(config, forward, series, horizon, context_length=None, cross_learning=False, max_output_patches=None,
             unrolled=(0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9), batch_size=256, max_tokens=131072):
    """Chronos2Pipeline.forecast. `config` needs context_length, patch_size, use_reg_token and the
    quantile levels (`quantiles`); series are (targets [V][T], past [V][T] or None, known [V][>=T+H]
    or None) tuples. Returns a list of [targets][Q][horizon] float32 arrays."""
    ps = config.patch_size
    levels = [f32(q) for q in config.quantiles]
    q = len(levels)
    cap = config.context_length
    ctx = min(context_length if context_length is not None else cap, cap)
    mop = max_output_patches if max_output_patches is not None else config.max_output_patches
    unrolled = [f32(u) for u in unrolled]

    def output_patches(remaining):
        return min((remaining + ps - 1) // ps, mop)

    def run(context, group, future, op):
        length = len(context[0])
        per_row = (min(length, cap) + ps - 1) // ps + (1 if config.use_reg_token else 0) + op
        if per_row * len(context) <= max_tokens:
            return forward(context, group, future, op)
        by_group = {}
        for i, g in enumerate(group):
            by_group.setdefault(g, []).append(i)
        out = [None] * len(context)
        chunk = []

        def run_chunk(rows):
            idx = sorted(rows)
            r = forward([context[i] for i in idx], [group[i] for i in idx], [future[i] for i in idx], op)
            for k, i in enumerate(idx):
                out[i] = r[k]

        for members in by_group.values():
            if chunk and (len(chunk) + len(members)) * per_row > max_tokens:
                run_chunk(chunk)
                chunk = []
            chunk.extend(members)
        run_chunk(chunk)
        return out

    def predict_step(context, group, future, op):
        size = op * ps
        f = []
        for row in future:
            n = min(size, len(row))
            f.append([f32(row[t]) for t in range(n)] + [f32(np.nan)] * (size - n))
        return run(context, group, f, op)

    def unroll(context, group, future, prediction, weights, op):
        rows, h, paths = len(prediction), len(prediction[0][0]), len(unrolled)
        values, lv = [], []
        for b in range(rows):
            for t in range(h):
                values.append([prediction[b][k][t] for k in range(q)])
                lv.append(levels)
        up = interpolate(unrolled, lv, values)
        length = min(len(context[0]) + h, cap)
        nxt, nfut = [None] * len(context), [None] * len(future)
        for b in range(rows):
            for n in range(paths):
                r = b * paths + n
                row = list(context[r]) + [up[b * h + t][n] for t in range(h)]
                row = row[len(row) - length:]
                f = future[r]
                for t in range(min(h, len(f))):
                    if not math.isnan(f[t]):
                        row[length - h + t] = f[t]
                nxt[r] = row
                nfut[r] = list(f[min(h, len(f)):])
        pred = predict_step(nxt, group, nfut, op)
        steps = len(pred[0][0])
        samples = []
        for b in range(rows):
            for t in range(steps):
                samples.append([pred[b * paths + n][k][t] for n in range(paths) for k in range(q)])
        merged = weighted_quantile(levels, weights, samples)
        out = [[[merged[b * steps + t][k] for t in range(steps)] for k in range(q)] for b in range(rows)]
        return out, nxt, nfut

    def predict_batch(batch):
        length = max(len(p[0][0]) for p in batch)
        context, future, group, first = [], [], [], []
        for s, (rows_c, rows_f, _t) in enumerate(batch):
            first.append(len(context))
            for i in range(len(rows_c)):
                context.append([f32(np.nan)] * (length - len(rows_c[i])) + list(rows_c[i]))
                future.append(rows_f[i])
                group.append(0 if cross_learning else s)
        rows = len(context)
        prediction = predict_step(context, group, future, output_patches(horizon))
        predictions = [prediction]
        remaining = horizon - len(prediction[0][0])
        if remaining > 0:
            paths = len(unrolled)
            context = [context[b] for b in range(rows) for _ in range(paths)]
            future = [future[b] for b in range(rows) for _ in range(paths)]
            group = [group[b] * paths + n for b in range(rows) for n in range(paths)]
            pm, lm = probability_mass(unrolled), probability_mass(levels)
            weights = [f32(pm[n] * lm[k]) for n in range(paths) for k in range(q)]
            while remaining > 0:
                prediction, context, future = unroll(context, group, future, prediction, weights,
                                                     output_patches(remaining))
                predictions.append(prediction)
                remaining -= len(prediction[0][0])
        out = []
        for s, (_c, _f, targets) in enumerate(batch):
            v = np.zeros((targets, q, horizon), np.float32)
            for t in range(targets):
                for k in range(q):
                    off = 0
                    for p in predictions:
                        src = p[first[s] + t][k]
                        n = min(len(src), horizon - off)
                        if n <= 0:
                            break
                        v[t, k, off: off + n] = np.asarray(src[:n], np.float32)
                        off += n
            out.append(v)
        return out

    prepared = []
    for target, past, known in series:
        length = len(target[0])
        keep = min(length, ctx)
        rows_c, rows_f = [], []
        for row in list(target) + ([] if past is None else list(past)):
            rows_c.append([f32(x) for x in row[length - keep: length]])
            rows_f.append([f32(np.nan)] * horizon)
        for row in ([] if known is None else list(known)):
            if len(row) < length + horizon:
                raise ValueError("future covariates too short")
            rows_c.append([f32(x) for x in row[length - keep: length]])
            rows_f.append([f32(x) for x in row[length: length + horizon]])
        prepared.append((rows_c, rows_f, len(target)))
    out = []
    start = 0
    while start < len(prepared):
        end, rows = start, 0
        while end < len(prepared) and rows < batch_size:
            rows += len(prepared[end][0])
            end += 1
        out.extend(predict_batch(prepared[start:end]))
        start = end
    return out
