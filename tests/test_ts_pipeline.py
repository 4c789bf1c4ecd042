"""Timestral's host pipeline (jitcast_amd.ts_pipeline) on the CPU.

Each piece is pinned by what the mathematics fixes: SeriesWindows by hand-counted windows, the sign
complement by symmetric and asymmetric level sets, target encoding by a hand-computed smoothed mean,
last_loc_scale by numpy's mean and Bessel-corrected std, the advancing refine frames by recomputing
every frame's mean and std from the values it folds in (two-pass, no Welford), the forward fill and
clamp_non_finite by small closed cases. The whole pipeline (windows, assembly, block decode with the
refine frames and the feedback, the cap, sign-flip averaging, the non-negative clip, categorical
covariates) is then checked against oracle/ts_pipeline.py, the reference's loops restated scalar by
scalar, over a deterministic stand-in block forward: every forward call's arguments and every forecast
must agree bit for bit. The reference's own golden vectors (scripts/timestral/dump_golden.py output)
are not in the repository, so the pipeline's parity with the upstream forecaster rests on these checks.
"""
import json
import math

import numpy as np
import pytest

from jitcast_amd import checkpoint as ck
from jitcast_amd import timestral_model as tm
from jitcast_amd import ts_pipeline as tp
from jitcast_amd.api import TimeSeries
from oracle import ts_pipeline as ref

f32 = np.float32
C = tm.TimestralConfig(patch_size=8, d_model=64, num_heads=2, mlp_hidden_dim=96, layers=((True, False), (True, False)),
                       quantiles=(0.1, 0.3, 0.5, 0.7, 0.9), block_size=4, context_length=96)


def test_split_windows_by_count_and_tokens():
    s = [TimeSeries.univariate(np.zeros(5))] * 5 + [TimeSeries([np.zeros(5)] * 3)]
    assert tp.split_windows(s, 2, 10**9, 4) == [(0, 2), (2, 4), (4, 6)]
    # 4 patches per row: tokens 4, 4, 4, 4, 4, 12; a budget of 9 holds two univariate series
    assert tp.split_windows(s, 100, 9, 4) == [(0, 2), (2, 4), (4, 5), (5, 6)]
    # a series over the budget runs alone
    assert tp.split_windows(s[5:], 100, 1, 4) == [(0, 1)]


def test_sign_complement():
    assert tp.sign_complement((0.1, 0.3, 0.5, 0.7, 0.9)).tolist() == [4, 3, 2, 1, 0]
    with pytest.raises(RuntimeError):
        tp.sign_complement((0.1, 0.5, 0.8))


def test_target_encoding_closed_form():
    t = np.array([1, 2, 3, 4], np.float32)
    codes = np.array([7, 9, 7, math.nan, 9, 11])  # context 4 steps, horizon 2: a seen code and an unseen one
    ts = TimeSeries([t], future_categorical=[codes])
    enc = tp.target_encode(ts, 2, 100)
    mean = 2.5
    exp = [(mean + 1 + 3) / 3, (mean + 2) / 2, (mean + 1 + 3) / 3, (mean + 4) / 2, (mean + 2) / 2, mean]
    np.testing.assert_array_equal(enc.future_covariates[0], np.asarray(exp, np.float64).astype(np.float32))
    # a missing code before the target starts is padding, not the missing category
    t2 = np.array([math.nan, 2, 4], np.float32)
    enc2 = tp.target_encode(TimeSeries([t2], past_categorical=[np.array([math.nan, 1, math.nan])]), 1, 100)
    v = enc2.past_covariates[0]
    assert math.isnan(v[0]) and v[1] == f32((3 + 2) / 2) and v[2] == f32((3 + 4) / 2)
    # two targets: the codes pass through
    enc3 = tp.target_encode(TimeSeries([t, t], past_categorical=[np.array([5, 6, 7, 8])]), 1, 100)
    np.testing.assert_array_equal(enc3.past_covariates[0], np.array([5, 6, 7, 8], np.float32))


def test_last_loc_scale_is_the_mean_and_bessel_std():
    r = np.random.default_rng(0)
    x = r.standard_normal((5, 64)).astype(np.float32) * 3 + 1
    obs = r.random((5, 64)) > 0.3
    loc, scale = tp.last_loc_scale(x, obs, 1e-6)
    for i in range(5):
        v = x[i][obs[i]].astype(np.float64)
        assert abs(loc[i] - v.mean()) <= 1e-6 * abs(v.mean()) + 1e-7
        assert abs(scale[i] - v.std(ddof=1)) <= 1e-6 * v.std(ddof=1)
    # no observation: loc 0, the floor as scale
    loc0, s0 = tp.last_loc_scale(np.ones((1, 8), np.float32), np.zeros((1, 8), bool), 0.25)
    assert loc0[0] == 0 and s0[0] == f32(0.25)


def test_advancing_frames_recomputed_two_pass():
    """Frame h holds the mean and std (ddof 1) of the observed context plus patches 0..h-1 of the
    block's median, each denormalised in its own frame: recomputed here from the values themselves."""
    r = np.random.default_rng(1)
    ps, t, hp = 8, 40, 4
    ctx = r.standard_normal((3, t)).astype(np.float32) * 2 + 5
    obs = r.random((3, t)) > 0.2
    sinh = r.standard_normal((3, hp, ps))
    locs, scales = tp.advancing_frames(ctx, obs, sinh, ps, 1e-6)
    for i in range(3):
        vals = list(ctx[i][obs[i]].astype(np.float64))
        for h in range(hp):
            v = np.asarray(vals)
            mu, sd = v.mean(), v.std(ddof=1)
            assert abs(locs[i, h] - mu) <= 1e-12 * max(1.0, abs(mu))
            assert abs(scales[i, h] - sd) <= 1e-12 * max(1.0, sd)
            vals += list(sinh[i, h] * sd + mu)


def test_native_statistics_equal_the_scalar_loops():
    """jc_ts_context_stats and jc_ts_advancing_frames (the library's host helpers behind last_loc_scale,
    the cap range and advancing_frames) against the restatement's scalar loops, value for value, on
    rows with gaps, NaN and +-inf, unobserved rows, one-step patches and scales from 1e-3 to 1e20
    (NaN compared as NaN, +0 and -0 as equal)."""
    r = np.random.default_rng(7)
    for trial in range(120):
        rows, patch = int(r.integers(1, 5)), int(r.choice([1, 2, 4, 16]))
        t = patch * int(r.integers(1, 30))
        x = (r.standard_normal((rows, t)) * r.choice([1e-3, 1, 1e3, 1e20])).astype(np.float32) + f32(r.standard_normal())
        obs = r.random((rows, t)) > r.choice([0.0, 0.3, 0.9, 1.0])
        if trial % 7 == 0:
            x[r.random((rows, t)) < 0.05] = np.nan
        if trial % 11 == 0:
            x[r.random((rows, t)) < 0.05] = np.inf
        ms = float(r.choice([1e-6, 1e-3, 0.5]))
        loc, scale, lo, hi = tp.context_stats(x, obs, ms)
        for i in range(rows):
            want = ref.last_loc_scale(x[i], obs[i], ms)
            np.testing.assert_array_equal([loc[i], scale[i]], np.asarray(want, np.float32))
            seen = x[i][obs[i]]
            np.testing.assert_array_equal([lo[i], hi[i]], [seen.min() if seen.size else 0, seen.max() if seen.size else 0])
        n_pred = int(r.integers(1, 6))
        sinh = r.standard_normal((rows, n_pred, patch)) * r.choice([1, 1e3, 1e30])
        if trial % 5 == 0:
            sinh[0, 0, 0] = np.nan
        locs, scales = tp.advancing_frames(x, obs, sinh, patch, ms)
        for i in range(rows):
            want = ref.advancing_frames(x[i], obs[i], sinh[i], patch, ms)
            np.testing.assert_array_equal(locs[i], want[0])
            np.testing.assert_array_equal(scales[i], want[1])


def test_native_statistics_threaded_equal_row_by_row():
    """Past 2^18 values the helpers split the rows over host threads: the same bits as each row
    computed alone (a single-threaded call)."""
    r = np.random.default_rng(9)
    rows, t, ps, hp = 64, 8192, 16, 4
    x = (r.standard_normal((rows, t)) * 5 + 2).astype(np.float32)
    obs = r.random((rows, t)) > 0.2
    sinh = r.standard_normal((rows, hp, ps))
    many = tp.context_stats(x, obs, 1e-6)
    frames = tp.advancing_frames(x, obs, sinh, ps, 1e-6)
    for i in range(0, rows, 7):
        one = tp.context_stats(x[i:i + 1], obs[i:i + 1], 1e-6)
        for a, b in zip(many, one):
            assert a[i].tobytes() == b[0].tobytes()
        f1 = tp.advancing_frames(x[i:i + 1], obs[i:i + 1], sinh[i:i + 1], ps, 1e-6)
        assert frames[0][i].tobytes() == f1[0][0].tobytes() and frames[1][i].tobytes() == f1[1][0].tobytes()


def test_native_statistics_reject_bad_shapes():
    """The host helpers return JC_EINVAL (raised as JitcastArgumentError) instead of reading past
    their arguments: a context shorter than one patch or not a whole number of patches, a patch below
    1, and a mask that does not match the values."""
    from jitcast_amd._lib import JitcastArgumentError

    x = np.ones((2, 12), np.float32)
    obs = np.ones((2, 12), bool)
    sinh = np.zeros((2, 1, 8))
    with pytest.raises(JitcastArgumentError):
        tp.advancing_frames(x[:, :4], obs[:, :4], sinh, 8, 1e-6)  # t < patch
    with pytest.raises(JitcastArgumentError):
        tp.advancing_frames(x, obs, sinh, 8, 1e-6)  # 12 steps is not a whole number of 8-step patches
    with pytest.raises(JitcastArgumentError):
        tp.advancing_frames(x[:, :8], obs[:, :8], np.zeros((2, 1, 0)), 0, 1e-6)  # patch 0
    with pytest.raises(ValueError):
        tp.context_stats(x, obs[:, :6], 1e-6)
    loc, scale, lo, hi = tp.context_stats(np.zeros((0, 5), np.float32), np.zeros((0, 5), bool), 1e-6)
    assert loc.shape == scale.shape == lo.shape == hi.shape == (0,)


def test_forward_fill_and_clamp_non_finite():
    x = np.array([0, 0, 3, 0, 5, 0], np.float32)
    m = np.array([False, False, True, False, True, False])
    np.testing.assert_array_equal(tp.forward_fill(x, m), [0, 0, 3, 3, 5, 5])
    v = np.array([[1, np.inf, -np.inf, 2], [np.inf, np.inf, np.nan, -np.inf]], np.float32)
    got = tp.clamp_non_finite(v)
    np.testing.assert_array_equal(got[0], [1, 2, 1, 2])
    assert got[1][0] == 0 and got[1][1] == 0 and math.isnan(got[1][2]) and got[1][3] == 0


# ---- the pipeline against the scalar restatement ------------------------------------------------

def fake_forward(c):
    """A deterministic stand-in for BlockForward.predictBlock: each row's quantiles from its last
    observed value, its observed mean, the step and the level; known rows' future enters too."""
    levels = np.asarray(c.quantiles, np.float32)

    def fwd(inputs, observed, group, h, role, kf, kfm):
        inputs = np.asarray(inputs, np.float32)
        observed = np.asarray(observed, bool)
        rows, t = inputs.shape
        n = h * c.patch_size
        out = np.empty((rows, n, levels.size), np.float32)
        for i in range(rows):
            o = np.nonzero(observed[i])[0]
            last = inputs[i, o[-1]] if o.size else f32(0)
            mean = f32(inputs[i, o].astype(np.float64).mean()) if o.size else f32(0)
            extra = f32(0)
            if kf is not None:
                extra = f32(np.asarray(kf[i], np.float64).sum() * 0.01)
            for s in range(n):
                base = f32(last + f32(0.05) * f32(s + 1) * (mean - last) + extra + f32(group[i]) * f32(0.001))
                out[i, s] = base + (levels - f32(0.5)) * f32(1 + 0.1 * s) * f32(1 + abs(float(mean)) * 0.1)
        return out

    return fwd


class Recorder:
    def __init__(self, fwd):
        self.fwd, self.calls = fwd, []

    def __call__(self, *a):
        self.calls.append([None if x is None else np.array(x, copy=True) for x in a])
        return self.fwd(*a)


def _series():
    r = np.random.default_rng(5)
    out = []
    # univariate, late start and a gap
    a = (r.standard_normal(70) + 3).astype(np.float32)
    a[:9] = np.nan
    a[30:33] = np.nan
    out.append(TimeSeries.univariate(a))
    # bivariate target, non-negative (clipped), with a past covariate
    b = np.abs(r.standard_normal((2, 50))).astype(np.float32)
    out.append(TimeSeries(b, past_covariates=[r.standard_normal(50)]))
    # known covariate with missing future values, and categorical past and known covariates
    cl = (np.sin(np.arange(64) / 4) * 2 - 1).astype(np.float32)
    fut = r.standard_normal(64 + 40).astype(np.float32)
    fut[70:73] = np.nan
    pc = r.integers(0, 3, 64).astype(np.float64)
    pc[5] = np.nan
    kc = r.integers(0, 4, 64 + 40).astype(np.float64)
    out.append(TimeSeries([cl], future_covariates=[fut], past_categorical=[pc], future_categorical=[kc]))
    # a long series (over the context cap) of one value plus noise
    out.append(TimeSeries.univariate((r.standard_normal(140) * 0.1 + 7).astype(np.float32)))
    return out


def _as_ref(ts):
    return {"target": list(ts.target), "past": None if ts.past_covariates is None else list(ts.past_covariates),
            "future": None if ts.future_covariates is None else list(ts.future_covariates),
            "pcat": None if ts.past_categorical is None else list(ts.past_categorical),
            "fcat": None if ts.future_categorical is None else list(ts.future_categorical)}


def _ref_config(c):
    return {"patch_size": c.patch_size, "block_size": c.block_size, "median": c.median_index,
            "num_quantiles": c.num_quantiles, "quantiles": c.quantiles, "minimum_scale": c.minimum_scale}


def _ref_options(o):
    return {"max_context": o.max_context, "per_shot": o.per_shot_horizon_patches, "cap_k": o.cap_k,
            "extreme": o.extreme_value_threshold, "symmetric": o.symmetric_averaging, "clip": o.clip_nonnegative}


@pytest.mark.parametrize("horizon,per_shot,symmetric,max_tokens", [(40, 2, True, 10**9), (13, 4, False, 10**9),
                                                                    (40, 2, True, 60), (8, 32, True, 10**9)])
def test_pipeline_matches_the_scalar_restatement(horizon, per_shot, symmetric, max_tokens):
    series = _series()
    o = tp.Options.defaults(C)
    o = tp.Options(o.max_context, per_shot, o.cap_k, o.extreme_value_threshold, symmetric, True)
    mine, theirs = Recorder(fake_forward(C)), Recorder(fake_forward(C))
    got = tp.TimestralPipeline(C, mine, o, max_tokens=max_tokens).forecast(series, horizon)
    exp = ref.forecast(_ref_config(C), _ref_options(o), theirs, [_as_ref(s) for s in series], horizon,
                       max_tokens=max_tokens)
    assert len(mine.calls) == len(theirs.calls) and len(mine.calls) > 0
    blocks = -(-horizon // C.patch_size)
    assert len(mine.calls) >= (2 if symmetric else 1) * -(-blocks // min(per_shot, C.block_size))
    for k, (a, b) in enumerate(zip(mine.calls, theirs.calls)):
        for name, x, y in zip(("inputs", "observed", "group", "h", "role", "kf", "kfm"), a, b):
            assert (x is None) == (y is None), (k, name)
            if x is not None:
                np.testing.assert_array_equal(np.asarray(x), np.asarray(y), err_msg=f"call {k} {name}")
    assert len(got) == len(series)
    for s, (g, e) in enumerate(zip(got, exp)):
        assert g.values.shape == e.shape == (series[s].targets(), C.num_quantiles, horizon)
        np.testing.assert_array_equal(g.values, e, err_msg=f"series {s}")
        np.testing.assert_array_equal(g.levels, np.asarray(C.quantiles, np.float32))
    # the non-negative bivariate series is clipped at 0
    assert (got[1].values >= 0).all()


def test_symmetric_forward_gives_an_odd_forecast():
    """With sign-flip averaging on, a forward that commutes with negation (quantile levels mirrored)
    makes forecast(-x) = -mirror(forecast(x)); the cap and clip are off for this check."""
    c = C
    levels = np.asarray(c.quantiles, np.float32)

    def odd(inputs, observed, group, h, role, kf, kfm):
        inputs = np.asarray(inputs, np.float32)
        n = h * c.patch_size
        last = inputs[:, -1:]
        return (np.repeat(last[:, :, None], n, axis=1) * f32(0.9)
                + (levels - f32(0.5))[None, None, :] * f32(2)).astype(np.float32)

    o = tp.Options(64, 4, 0.0, 1e30, True, False)
    p = tp.TimestralPipeline(c, odd, o)
    x = (np.random.default_rng(2).standard_normal(40) + 1).astype(np.float32)
    a = p.forecast([TimeSeries.univariate(x)], 16)[0].values
    b = p.forecast([TimeSeries.univariate(-x)], 16)[0].values
    np.testing.assert_allclose(a, -b[:, ::-1], rtol=0, atol=1e-6)


def test_pipeline_rejects_what_the_reference_rejects():
    p = tp.TimestralPipeline(C, fake_forward(C))
    with pytest.raises(ValueError):
        p.forecast([TimeSeries.univariate(np.ones(10))], 0)
    no_cov = tm.TimestralConfig(**{**C.__dict__, "covariate_enabled": False})
    with pytest.raises(ValueError, match="covariates"):
        tp.TimestralPipeline(no_cov, fake_forward(no_cov)).forecast(
            [TimeSeries([np.ones(10)], past_covariates=[np.ones(10)])], 4)
    time_only = tm.TimestralConfig(**{**C.__dict__, "layers": ((True,), (True,))})
    with pytest.raises(ValueError, match="known-future"):
        tp.TimestralPipeline(time_only, fake_forward(time_only)).forecast(
            [TimeSeries([np.ones(10)], future_covariates=[np.ones(20)])], 4)
    with pytest.raises(ValueError, match="at least"):
        p.forecast([TimeSeries([np.ones(10)], future_covariates=[np.ones(12)])], 4)
    with pytest.raises(ValueError):
        tp.TimestralPipeline(C, fake_forward(C), tp.Options(4, 4, 1.0, 1e30, True, True))


# ---- checkpoints ---------------------------------------------------------------------------------

def test_checkpoint_round_trip_and_layouts(tmp_path):
    w = tm.random_weights(C, seed=3)
    ck.write_timestral(tmp_path, C, w)
    c2, w2 = ck.load_timestral(tmp_path)
    assert c2.layers == C.layers and c2.quantiles == C.quantiles and c2.context_length == C.context_length
    assert c2.norm_eps == float(f32(C.norm_eps))
    for la, lb in zip(w["layers"], w2["layers"]):
        for aa, ab in zip(la["attentions"], lb["attentions"]):
            for k in ("norm", "qkv", "gate", "wo"):
                np.testing.assert_array_equal(aa[k], ab[k])
        for k in ("mlp_norm", "up", "down"):
            np.testing.assert_array_equal(la[k], lb[k])
    for k in ("query", "out_norm", "embed_hidden_w", "embed_hidden_b", "head_output_w"):
        np.testing.assert_array_equal(w[k], w2[k])
    # on disk: wQKV row s*d + e*heads + h is engine row s*d + h*dh + e; w12's halves exchanged
    with ck.SafeTensors(tmp_path / "model.safetensors") as st:
        raw = st.get("transformer.layers.1.attns.0.wQKV.weight").to_numpy()
        up = st.get("transformer.layers.1.mlp.w12.weight").to_numpy()
    d, heads, dh, f = C.d_model, C.num_heads, C.head_dim, C.mlp_hidden_dim
    eng = w["layers"][1]["attentions"][0]["qkv"]
    for s in range(3):
        for h in range(heads):
            np.testing.assert_array_equal(raw[s * d + np.arange(dh) * heads + h], eng[s * d + h * dh:s * d + (h + 1) * dh])
    np.testing.assert_array_equal(up[:f], w["layers"][1]["up"][f:])


@pytest.mark.parametrize("edit,match", [
    (lambda d: d.update(extra=1), "unknown config key"),
    (lambda d: d.update(attn_bias=True), "attn_bias"),
    (lambda d: d.update(time_attn_gate="softmax"), "gate"),
    (lambda d: d.update(block_schedule=["time", "cross"]), "layer kind"),
    (lambda d: d.update(quantile_knots=[0.5, 0.1]), "increasing"),
    (lambda d: d.update(quantile_knots=[0.1, 0.9]), "0.5"),
    (lambda d: d.update(context_length=100), "multiple"),
])
def test_config_is_parsed_strictly(edit, match):
    doc = json.loads(ck.ts_config_json(C))
    edit(doc)
    with pytest.raises(ValueError, match=match):
        ck.parse_ts_config(json.dumps(doc))


def test_tensors_are_bound_exactly(tmp_path):
    w = tm.random_weights(C, seed=4)
    ck.write_timestral(tmp_path, C, w)
    tensors = {}
    with ck.SafeTensors(tmp_path / "model.safetensors") as st:
        for name in st.tensors:
            tensors[name] = st.get(name).to_numpy().copy()
    for change, match in ((lambda t: t.pop("transformer.out_norm.scale"), "no tensor"),
                          (lambda t: t.update(extra=np.zeros(3, np.float32)), "unexpected"),
                          (lambda t: t.update({"representation.forecast_query": np.zeros(5, np.float32)}), None)):
        t = dict(tensors)
        change(t)
        ck.write_safetensors(tmp_path / "model.safetensors", t)
        with pytest.raises(ValueError, match=match):
            ck.load_timestral(tmp_path)
