"""The Chronos-2 host pipeline (jitcast_amd.pipeline, jitcast_amd.quantile_math) on the CPU.

- QuantileMath is pinned by closed forms (uniform masses, identity at the knots, exact linear
  interpolation, the order statistics of an equally weighted sample, the batch-wide end-point rule,
  Float.compare's order) and agrees bit for bit with the oracle's scalar restatement.
- Every forward call the pipeline makes, and the forecasts, equal bit for bit those of the oracle's
  loop-by-loop restatement of Chronos2Pipeline (oracle/c2_pipeline.py) over the same forward pass, on
  the reference's mixed-batch recipe (Chronos2BatchParityAccelTest.java:64-108: ragged lengths, late
  starts, gaps, past-only and known covariates, a horizon that unrolls), on many tiny series across
  several batches, with cross-learning, past the context cap, and split by the token budget
  (PipelineGoldenTest.java:45-104 compares calls the same way against the reference's recordings).
The forward pass here is a deterministic stand-in (row-wise, so token-budget splits cannot change
it); the HIP forward under this pipeline is checked against the oracle in tests/test_gpu_engine.py.
"""
import math

import numpy as np
import pytest

from jitcast_amd import quantile_math as qm
from jitcast_amd.api import Forecast, TimeSeries
from jitcast_amd.chronos2_model import Chronos2Config
from jitcast_amd.pipeline import Chronos2Pipeline, Options
from oracle import c2_pipeline as ref

SMALL = Chronos2Config(d_model=64, d_kv=16, d_ff=128, num_layers=2, num_heads=4, context_length=512, patch_size=16,
                       max_output_patches=4, time_encoding_scale=512)


# ---- QuantileMath ------------------------------------------------------------------------------

def test_probability_mass_closed_forms():
    m = qm.probability_mass([0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9])
    np.testing.assert_allclose(m, np.full(9, 1 / 9), rtol=1e-6)
    m21 = qm.probability_mass(SMALL.quantile_levels())
    assert abs(float(m21.astype(np.float64).sum()) - 1) < 1e-6
    # the ends: (0.05 - 0) / 2 and (1 - 0.95) / 2 before normalizing
    raw = np.array([0.025, 0.045, 0.05], np.float64)
    np.testing.assert_allclose(m21[:3] / m21[1], raw / raw[1], rtol=1e-5)
    np.testing.assert_array_equal(m, np.asarray(ref.probability_mass([0.1 * (i + 1) for i in range(9)]), np.float32))


def test_interpolate_is_exact_at_the_knots_and_linear_between():
    levels = SMALL.quantile_levels()
    r = np.random.default_rng(0)
    vals = np.sort(r.standard_normal((50, levels.size)).astype(np.float32), axis=1)
    np.testing.assert_array_equal(qm.interpolate(levels, levels, vals), vals)
    # values linear in the level: interpolation reproduces the line inside the knots
    a, b = np.float32(3.0), np.float32(-2.0)
    lin = (a + b * levels)[None, :].repeat(4, axis=0).astype(np.float32)
    query = np.array([0.01, 0.033, 0.5, 0.77, 0.99], np.float32)
    np.testing.assert_allclose(qm.interpolate(query, levels, lin), np.broadcast_to(a + b * query, (4, 5)), atol=1e-6)
    # beyond the lowest and highest level the end values extend flat to 0 and 1
    out = qm.interpolate(np.array([0.0, 0.005, 0.995, 1.0], np.float32), levels, lin)
    np.testing.assert_array_equal(out[:, :2], lin[:, :1].repeat(2, axis=1))
    np.testing.assert_array_equal(out[:, 2:], lin[:, -1:].repeat(2, axis=1))


def test_interpolate_end_points_are_decided_for_the_whole_batch():
    """One row holding level 0 removes the low end point for every row (QuantileMath.java:55-62)."""
    levels = np.array([[0.0, 0.5, 1.0], [0.25, 0.5, 0.75]], np.float32)
    vals = np.array([[0.0, 5.0, 10.0], [1.0, 2.0, 3.0]], np.float32)
    out = qm.interpolate(np.array([0.1], np.float32), levels, vals)
    # row 1 without the 0-level end point: below 0.25 it extrapolates the first segment's line
    # (lower = upper = index 0 gives w = 0/0 -> 0, so the value is the first value)
    assert out[1, 0] == np.float32(1.0)
    assert out[0, 0] == np.float32(1.0)  # 0.1 of the way from 0 to 10 over [0, 0.5]... 0.2 * 5
    np.testing.assert_array_equal(out, np.asarray(ref.interpolate([0.1], levels.tolist(), vals.tolist()), np.float32))


def test_weighted_quantile_of_equal_weights_is_the_order_statistic():
    r = np.random.default_rng(1)
    s = r.standard_normal((20, 4)).astype(np.float32)
    out = qm.weighted_quantile(np.array([0.25, 0.5, 0.75, 1.0], np.float32), np.ones(4, np.float32), s)
    # levels 1/4, 2/4, 3/4 hit a knot (weight 0 on the next value): exact
    np.testing.assert_array_equal(out[:, :3], np.sort(s, axis=1)[:, :3])
    # level 1 is reached as v3 + 1 * (v4 - v3), within one rounding of v4
    np.testing.assert_allclose(out[:, 3], np.sort(s, axis=1)[:, 3], rtol=0, atol=2e-7)


def test_float_compare_order():
    v = np.array([np.nan, 0.0, -0.0, -np.inf, 1.0, np.inf, -1.0, np.float32(-np.nan)], np.float32)
    order = np.argsort(qm.float_compare_key(v), kind="stable")
    assert [repr(float(x)) for x in v[order][:6]] == ["-inf", "-1.0", "-0.0", "0.0", "1.0", "inf"]
    assert np.isnan(v[order][6:]).all() and list(order[6:]) == [0, 7]
    assert sorted(range(8), key=lambda i: ref._fc_key(v[i])) == list(order)


def test_quantile_math_matches_the_scalar_restatement():
    r = np.random.default_rng(2)
    levels = SMALL.quantile_levels()
    vals = r.standard_normal((64, levels.size)).astype(np.float32)
    vals[3, 4] = np.nan
    vals[5, :] = 0.0
    vals[6, 2] = -0.0
    unrolled = np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9], np.float32)
    got = qm.interpolate(unrolled, levels, vals)
    exp = np.asarray(ref.interpolate(unrolled, [levels] * 64, vals.tolist()), np.float32)
    np.testing.assert_array_equal(got, exp)
    w = (qm.probability_mass(unrolled)[:, None] * qm.probability_mass(levels)[None, :]).reshape(-1).astype(np.float32)
    samples = r.standard_normal((40, w.size)).astype(np.float32)
    samples[0, 7] = np.nan
    got = qm.weighted_quantile(levels, w, samples)
    exp = np.asarray(ref.weighted_quantile(levels, w.tolist(), samples.tolist()), np.float32)
    np.testing.assert_array_equal(got, exp)


# ---- the pipeline's forward calls ------------------------------------------------------------

def _stand_in(c):
    """A deterministic row-wise forward: each row's quantiles from the mean and spread of its last
    observed steps and its known future values, in float32."""
    levels = c.quantile_levels()

    def fwd(context, group, future, op):
        ctx = np.asarray(context, np.float32)
        fut = np.asarray(future, np.float32)
        steps = op * c.patch_size
        tail = ctx[:, -32:]
        with np.errstate(all="ignore"):
            obs = ~np.isnan(tail)
            mean = np.where(obs, tail, 0).sum(axis=1) / np.maximum(obs.sum(axis=1), 1)
            spread = 0.1 + np.abs(np.where(obs, tail - mean[:, None], 0)).sum(axis=1) / np.maximum(obs.sum(axis=1), 1)
        mean, spread = mean.astype(np.float32), spread.astype(np.float32)
        t = np.arange(steps, dtype=np.float32)
        f = np.nan_to_num(fut, nan=0.0).astype(np.float32)
        g = np.asarray(group, np.float32)[:, None, None] * np.float32(1e-3)
        out = (mean[:, None, None] + spread[:, None, None] * (levels[None, :, None] - np.float32(0.5)) * np.float32(4)
               + np.float32(0.01) * t[None, None, :] + np.float32(0.5) * f[:, None, :] + g)
        return out.astype(np.float32)

    return fwd


def _recording(fwd, calls):
    def f(inp):
        calls.append((inp.context.copy(), inp.group.copy(), inp.future_covariates.copy(), inp.output_patches))
        return fwd(inp.context, inp.group, inp.future_covariates, inp.output_patches)

    return f


def _recording_ref(fwd, calls):
    def f(context, group, future, op):
        calls.append((np.asarray(context, np.float32), np.asarray(group, np.int32), np.asarray(future, np.float32), op))
        return fwd(context, group, future, op)

    return f


def _mixed_batch(seed, count, horizon, walk_len=(40, 300)):
    """The reference's mixed batch (Chronos2BatchParityAccelTest.batch): random walks plus a daily
    cycle, every fifth series bivariate, late starts, gaps, past-only and 0/1 known covariates."""
    r = np.random.default_rng(seed)
    out = []
    for s in range(count):
        length = int(r.integers(walk_len[0], walk_len[1]))
        targets = 2 if s % 5 == 0 else 1

        def walk(rows):
            w = np.empty((rows, length), np.float32)
            for i in range(rows):
                v = 10 * r.random() + np.cumsum(r.standard_normal(length) * 0.3)
                w[i] = v + 2 * np.sin(2 * np.pi * np.arange(length) / 24)
            return w

        t = walk(targets)
        if s % 7 == 3:
            t[0, : min(length, 50)] = np.nan
        if s % 4 == 1:
            t[0, length // 3: length // 3 + 20] = np.nan
        past = walk(int(1 + r.integers(0, 2))) if s % 3 == 1 else None
        known = None
        if s % 3 == 2:
            known = np.tile(((np.arange(length + horizon) % 24) < 6).astype(np.float32), (int(1 + r.integers(0, 2)), 1))
        out.append((t, past, known))
    return out


def _compare(series, horizon, c=SMALL, **kw):
    fwd = _stand_in(c)
    got_calls, exp_calls = [], []
    pipe_kw = {k: v for k, v in kw.items() if k in ("batch_size", "max_tokens")}
    o = Options.defaults(c)
    if "cross_learning" in kw:
        o = o.with_cross_learning(kw["cross_learning"])
    if "context_length" in kw:
        o = o.with_context_length(kw["context_length"])
    p = Chronos2Pipeline(c, _recording(fwd, got_calls), o, **pipe_kw)
    got = p.forecast([TimeSeries(t, pc, k) for t, pc, k in series], horizon)
    exp = ref.forecast(c, _recording_ref(fwd, exp_calls), series, horizon, **kw)
    assert len(got_calls) == len(exp_calls)
    for (gc, gg, gf, go), (ec, eg, ef, eo) in zip(got_calls, exp_calls):
        assert go == eo
        np.testing.assert_array_equal(gc, ec)  # NaN where NaN, bit for bit elsewhere
        np.testing.assert_array_equal(gg, eg)
        np.testing.assert_array_equal(gf, ef)
    assert len(got) == len(series)
    for g, e, (t, _, _) in zip(got, exp, series):
        assert isinstance(g, Forecast)
        assert g.values.shape == (len(t), c.num_quantiles, horizon)
        np.testing.assert_array_equal(g.values, e)
        np.testing.assert_array_equal(g.levels, c.quantile_levels())
    return got_calls


def test_mixed_batch_unrolls_and_matches_the_restatement():
    calls = _compare(_mixed_batch(11, 25, 100), 100)
    # 4 patches per pass: 64 steps, then the unrolled pass over 9 paths per row
    assert [c[3] for c in calls] == [4, 3]
    assert calls[1][0].shape[0] == 9 * calls[0][0].shape[0]
    # a group of the unrolled pass holds one path of one series: its rows are not adjacent
    g = calls[1][1]
    assert g[0] != g[1] and np.count_nonzero(g == g[0]) == np.count_nonzero(calls[0][1] == calls[0][1][0])


def test_many_tiny_series_span_batches():
    series = [(np.asarray([np.linspace(0, 1, 5 + i % 7)], np.float32), None, None) for i in range(300)]
    calls = _compare(series, 20, batch_size=64)
    assert len(calls) == 5 and [c[0].shape[0] for c in calls] == [64, 64, 64, 64, 44]


def test_cross_learning_puts_a_batch_in_one_group():
    calls = _compare(_mixed_batch(3, 8, 30), 30, cross_learning=True)
    assert (calls[0][1] == 0).all()


def test_context_cap_keeps_the_latest_steps():
    long = np.sin(np.arange(600, dtype=np.float32) / 7)[None, :]
    calls = _compare([(long, None, None), (long[:, :100], None, None)], 16)
    assert calls[0][0].shape == (2, 512)
    np.testing.assert_array_equal(calls[0][0][0], long[0, -512:])
    assert np.isnan(calls[0][0][1, :412]).all()
    calls = _compare([(long, None, None)], 16, context_length=200)
    assert calls[0][0].shape == (1, 200)


def test_token_budget_splits_passes_by_whole_groups():
    series = _mixed_batch(5, 12, 100)
    one = _compare(series, 100)
    split = _compare(series, 100, max_tokens=300)
    assert len(split) > len(one)
    # no group is split across passes: each pass holds all of a group's rows of the unsplit pass
    for ctx, grp, _, op in split:
        full = next(g for c, g, _, o in one if o == op)
        for gid in np.unique(grp):
            assert np.count_nonzero(grp == gid) == np.count_nonzero(full == gid)
    fwd = _stand_in(SMALL)
    a = Chronos2Pipeline(SMALL, _recording(fwd, []), max_tokens=300).forecast(
        [TimeSeries(t, p, k) for t, p, k in series], 100)
    b = Chronos2Pipeline(SMALL, _recording(fwd, [])).forecast([TimeSeries(t, p, k) for t, p, k in series], 100)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x.values, y.values)


def test_pipeline_rejects_what_the_reference_rejects():
    fwd = _recording(_stand_in(SMALL), [])
    p = Chronos2Pipeline(SMALL, fwd)
    with pytest.raises(ValueError, match="horizon"):
        p.forecast([TimeSeries.univariate(np.ones(10))], 0)
    with pytest.raises(ValueError, match="categorical"):
        p.forecast([TimeSeries([np.ones(10)], past_categorical=[np.zeros(10)])], 4)
    with pytest.raises(ValueError, match="future covariates need"):
        p.forecast([TimeSeries([np.ones(10)], None, [np.ones(12)])], 4)
    with pytest.raises(ValueError, match="unrolled quantile"):
        Chronos2Pipeline(SMALL, fwd, Options(512, False, 4, (0.12,)))
    with pytest.raises(ValueError):
        Chronos2Pipeline(SMALL, fwd, batch_size=0)


def test_time_series_checks_shapes():
    """TimeSeriesTest.java: no time steps, covariates of another length."""
    with pytest.raises(ValueError):
        TimeSeries.univariate(np.zeros(0, np.float32))
    with pytest.raises(ValueError):
        TimeSeries([[1, 2, 3]], [[1, 2]], None)
    with pytest.raises(ValueError):
        TimeSeries([[1, 2, 3]], None, [[1, 2]])
    with pytest.raises(ValueError):
        TimeSeries([[1, 2, 3]], past_categorical=[[1, math.inf, 2]])
    ts = TimeSeries([[1, 2, 3], [4, 5, 6]], [[0, 0, 0]], [[1, 1, 1, 1, 1]])
    assert (ts.length(), ts.targets(), ts.rows()) == (3, 2, 4)
    f = Forecast(np.array([0.1, 0.5, 0.9], np.float32), np.arange(12, dtype=np.float32).reshape(1, 3, 4))
    np.testing.assert_array_equal(f.median(0), [4, 5, 6, 7])
