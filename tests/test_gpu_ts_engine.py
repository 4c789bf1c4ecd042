"""GPU parity of the HIP Timestral engine (jitcast_amd.engine.HipTimestralEngine: a checkpoint loaded
from config.json + model.safetensors, TimestralPipeline on the host, predict_block on the device)
against the oracle: oracle/ts_pipeline.py's scalar restatement of TimestralPipeline over the oracle's
CpuTimestral.predictBlock restatement (its BlockLayout, BlockPrep, forward and finish).

The batch mixes what the pipeline handles: a late start and a gap, a bivariate target with a past
covariate, a known-future covariate with missing future steps and categorical past and known
covariates, and a series longer than the context cap. The horizon spans several blocks, so each block
is moved to the refine frame and its median fed back; sign-flip averaging doubles the passes. The first
forward call of each pass sees the assembled batch, which must equal the oracle's bit for bit; the
forecasts are held to the end-to-end bar of 1e-3.
"""
import numpy as np
import pytest

from jitcast_amd import checkpoint as ck
from jitcast_amd import timestral_model as tm
from jitcast_amd.api import TimeSeries
from jitcast_amd.engine import HipTimestralEngine
from oracle import ts_pipeline as ref
from tests.test_ts_pipeline import _as_ref, _ref_config, _ref_options, _series

pytestmark = pytest.mark.gpu

C = tm.TimestralConfig(patch_size=8, d_model=64, num_heads=2, mlp_hidden_dim=96, layers=((True, False), (True, False)),
                       quantiles=(0.1, 0.3, 0.5, 0.7, 0.9), block_size=4, context_length=96)


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    d = tmp_path_factory.mktemp("tsckpt")
    ck.write_timestral(d, C, tm.random_weights(C, seed=31, std=0.1))
    return d


def _oracle_forward(oracle, c, w, calls):
    def fwd(x, obs, group, h, role, fut, fut_mask):
        calls.append(np.array(x, copy=True))
        ps = c.patch_size
        window, wobs, enc, cov, kv, known, position, ll = oracle.ts_block_layout(
            x, obs, group, h, ps, role, fut, fut_mask, c.covariate_enabled, c.attend_missing, c.block_size)
        tok, _, loc, scale = oracle.ts_block_prep(window, wobs, known, ps, c.minimum_scale, c.use_asinh)
        rows = x.shape[0]
        raw = oracle.ts_forward_raw(tok, w, kv, known, position, group,
                                    np.asarray(role, np.int32) if cov else np.zeros(rows, np.int32), cov, rows, enc,
                                    ll, h, c.num_heads, c.head_dim, c.rope_dim, c.norm_eps, c.rope_theta)
        return oracle.ts_block_finish(raw, loc, scale, ll, h, ps, c.quantiles, c.median_index,
                                      c.quantile_width_factor, c.use_asinh)
    return fwd


@pytest.mark.parametrize("horizon,per_shot", [(40, 2), (13, 32)])
def test_engine_matches_the_oracle_pipeline(gpu, oracle, checkpoint, horizon, per_shot):
    print(f"case timestral engine horizon={horizon} per_shot={per_shot}", flush=True)
    series = _series()
    c, w = ck.load_timestral(checkpoint)
    with HipTimestralEngine.load(checkpoint, dtype="f32") as eng:
        o = eng.pipeline().options()
        pipe = eng.pipeline().with_options(type(o)(o.max_context, per_shot, o.cap_k, o.extreme_value_threshold,
                                                   o.symmetric_averaging, o.clip_nonnegative))
        mine = []
        fwd = pipe.forward
        pipe.forward = lambda x, *a: mine.append(np.array(x, copy=True)) or fwd(x, *a)
        got = pipe.forecast(series, horizon)
        theirs = []
        exp = ref.forecast(_ref_config(c), _ref_options(pipe.options()), _oracle_forward(oracle, c, w, theirs),
                           [_as_ref(s) for s in series], horizon)
    assert len(mine) == len(theirs)
    blocks = -(-(-(-horizon // c.patch_size)) // min(per_shot, c.block_size))
    np.testing.assert_array_equal(mine[0], theirs[0])  # the assembled batch of the first pass
    np.testing.assert_array_equal(mine[blocks], theirs[blocks])  # and of the mirrored pass
    err = max(oracle.rel_max_error(g.values, e) for g, e in zip(got, exp))
    print(f"  {len(mine)} block calls, forecasts rel err {err:.2e} (bar 1e-3)", flush=True)
    assert err <= 1e-3
    for g, s in zip(got, series):
        assert g.values.shape == (s.targets(), c.num_quantiles, horizon)
        assert np.all(np.diff(g.values, axis=1) >= -1e-6)  # quantiles do not cross


def test_engine_contract(gpu, checkpoint):
    """ForecastEngine's contract: a name, horizon checked, one Forecast per series in order with the
    model's levels, close() idempotent and final."""
    eng = HipTimestralEngine.load(checkpoint)
    assert eng.name() == "timestral-hip"
    with pytest.raises(ValueError):
        eng.forecast([TimeSeries.univariate(np.ones(20))], 0)
    out = eng.forecast([TimeSeries.univariate(np.arange(30, dtype=np.float32)),
                        TimeSeries.univariate(-np.arange(20, dtype=np.float32))], 5)
    assert len(out) == 2 and out[0].values.shape == (1, 5, 5)
    np.testing.assert_array_equal(out[1].levels, np.asarray(C.quantiles, np.float32))
    eng.close()
    eng.close()
    with pytest.raises(RuntimeError):
        eng.forecast([TimeSeries.univariate(np.ones(20))], 4)


@pytest.mark.parametrize("buckets", [True, False])
def test_capturing_forecast_equals_replayed(gpu, checkpoint, buckets):
    """A fresh engine's first forecast captures its plans, the second replays them: both bit for bit
    equal to the eager forward's (no plans), so neither a capture nor a replay reads or writes out of
    stream order."""
    print(f"case timestral engine capture vs replay buckets={buckets}", flush=True)
    series = _series()
    with HipTimestralEngine.load(checkpoint, dtype="f32", max_plans=0, buckets=buckets) as eager:
        want = eager.forecast(series, 40)
    with HipTimestralEngine.load(checkpoint, dtype="f32", max_plans=8, buckets=buckets) as eng:
        first = eng.forecast(series, 40)
        second = eng.forecast(series, 40)
        assert eng.forward_pass().plans.keys()
    for a, b, e in zip(first, second, want):
        np.testing.assert_array_equal(a.values, e.values)
        np.testing.assert_array_equal(b.values, e.values)


C_LONG = tm.TimestralConfig(patch_size=16, d_model=64, num_heads=2, mlp_hidden_dim=96,
                            layers=((True, False), (True, False)), quantiles=(0.1, 0.3, 0.5, 0.7, 0.9))


def _walk(r, rows: int, length: int) -> np.ndarray:
    v = 10 * r.random((rows, 1))
    steps = np.cumsum(0.3 * r.standard_normal((rows, length)), axis=1) + v
    return (steps + 2 * np.sin(2 * np.pi * np.arange(length) / 24)).astype(np.float32)


def _mixed_batch(seed: int, count: int, horizon: int) -> list:
    """The shape of TimestralBatchParityAccelTest.batch (TimestralBatchParityAccelTest.java:75-104):
    series of 40..939 steps, every fifth with two targets, late starts, gaps, past covariates on every
    third and known-future covariates (a daily on/off pattern) on another third."""
    r = np.random.default_rng(seed)
    out = []
    for s in range(count):
        length = 40 + int(r.integers(900))
        t = _walk(r, 2 if s % 5 == 0 else 1, length)
        if s % 7 == 3:
            t[0, :min(length, 50)] = np.nan  # a late start
        if s % 4 == 1:
            t[0, length // 3:length // 3 + 20] = np.nan  # a gap
        past = _walk(r, 1 + int(r.integers(2)), length) if s % 3 == 1 else None
        known = None
        if s % 3 == 2:
            row = ((np.arange(length + horizon) % 24) < 6).astype(np.float32)
            known = np.stack([row] * (1 + int(r.integers(2))))
        out.append(TimeSeries(t, past, known))
    return out


@pytest.fixture(scope="module")
def long_checkpoint(tmp_path_factory):
    d = tmp_path_factory.mktemp("tsckpt_long")
    ck.write_timestral(d, C_LONG, tm.random_weights(C_LONG, seed=5, std=0.1))
    return d


@pytest.mark.parametrize("dtype,bar", [("f32", 1e-4), ("f16x3", 1e-4), ("bf16", 5e-2), ("fp16", 5e-2)])
def test_mixed_batch_calls_match_the_oracle_forward(gpu, oracle, long_checkpoint, dtype, bar):
    """TimestralBatchParityAccelTest.mixedBatchMatchesTheCpuReference: 37 mixed series at horizon 1100
    (several blocks per pass, both sign passes), every predict_block call of the engine's pipeline
    against the oracle's block forward on the same inputs, within 1e-4 in fp32 and the reference's
    REDUCED_TOLERANCE (5e-2) with reduced-precision GEMMs."""
    horizon = 1100
    series = _mixed_batch(11, 37, horizon)
    c, w = ck.load_timestral(long_checkpoint)
    calls = []
    with HipTimestralEngine.load(long_checkpoint, dtype=dtype) as eng:
        pipe = eng.pipeline()
        fwd = pipe.forward

        def rec(*a):
            out = fwd(*a)
            calls.append(([None if x is None else np.array(x, copy=True) for x in a], np.array(out, copy=True)))
            return out

        pipe.forward = rec
        try:
            got = eng.forecast(series, horizon)
        finally:
            pipe.forward = fwd
    assert len(got) == len(series) and all(np.isfinite(f.values).all() for f in got)
    ofwd = _oracle_forward(oracle, c, w, [])
    worst = 0.0
    for k, (args, out) in enumerate(calls):
        x, obs, group, h, role, kf, kfm = args
        err = oracle.rel_max_error(out, ofwd(x, obs, group, int(h), role, kf, kfm))
        print(f"  mixed batch call{k} rows={x.shape[0]} length={x.shape[1]} horizon patches={int(h)} "
              f"covariates={role is not None} rel max err {err:.2e}", flush=True)
        worst = max(worst, err)
    assert len(calls) >= 6 and worst <= bar


def test_ragged_series_match_their_padded_batch(gpu, long_checkpoint):
    """PipelineGoldenTest.raggedSeriesMatchTheirPaddedBatch: series passed at their own lengths forecast
    as the same series left-padded with NaN to one length do (leading unobserved patches are never
    keys and positions count from each series' first observation), within 1e-4."""
    r = np.random.default_rng(4)
    lengths = (300, 173, 64, 250, 97, 300)
    ragged = [TimeSeries.univariate(_walk(r, 1, n)[0]) for n in lengths]
    padded = [TimeSeries.univariate(np.concatenate([np.full(300 - s.length(), np.nan, np.float32), s.target[0]]))
              for s in ragged]
    with HipTimestralEngine.load(long_checkpoint, dtype="f32") as eng:
        a = eng.forecast(ragged, 48)
        b = eng.forecast(padded, 48)
    err = max(float(np.max(np.abs(x.values - y.values)) / np.max(np.abs(y.values))) for x, y in zip(a, b))
    print(f"  ragged vs padded forecasts rel max err {err:.2e}", flush=True)
    assert err <= 1e-4
