"""Pins of the oracle's Timestral block forward (CpuTimestral.predictBlock from the patch tokens to the
head's raw outputs, J/timestral/cpu/CpuTimestral.java:127-188) and of its new pieces (Ops.silu, the
SwiGLU activation, the SiLU residual block) against closed forms and a float64 restatement built on
tests/brute.py's attention. CPU only."""
import numpy as np
import pytest

from jitcast_amd import timestral_model as tm
from tests import brute, cases

pytestmark = pytest.mark.usefixtures("oracle")

TINY = tm.TimestralConfig(patch_size=8, d_model=32, num_heads=2, mlp_hidden_dim=48,
                          layers=((True, False), (False, True)), quantiles=(0.1, 0.5, 0.9))


def test_silu_closed_forms(oracle):
    x = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 1e-8], np.float32)
    got = oracle.silu(x)
    exp = np.array([0.0, 1.0 / (1.0 + np.exp(-1.0)), -1.0 / (1.0 + np.exp(1.0)), 30.0, -30.0 * np.exp(-30.0) / (1 + np.exp(-30.0)),
                    5e-9], np.float64)
    np.testing.assert_allclose(got, exp.astype(np.float32), rtol=2e-7, atol=0)
    assert got[0] == 0 and got[3] == np.float32(30.0)


def test_swiglu_gate_half_first(oracle):
    """act = silu(first half) * second half: a unit second half returns silu of the first, a zero
    first half returns 0 whatever the second."""
    r = np.random.default_rng(0)
    a = r.standard_normal((5, 7)).astype(np.float32)
    up = np.concatenate([a, np.ones((5, 7), np.float32)], axis=1)
    np.testing.assert_array_equal(oracle.swiglu(up, 7), oracle.silu(a))
    up = np.concatenate([np.zeros((5, 7), np.float32), a], axis=1)
    np.testing.assert_array_equal(oracle.swiglu(up, 7), np.zeros((5, 7), np.float32))


def _lin(x, w, b=None):
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    return y if b is None else y + np.asarray(b, np.float64)


def _rms(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps) * np.asarray(w, np.float64)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _res(x, w, pre):
    hid = _silu(_lin(x, w[pre + "_hidden_w"], w.get(pre + "_hidden_b")))
    return _lin(hid, w[pre + "_output_w"], w.get(pre + "_output_b")) + _lin(x, w[pre + "_residual_w"],
                                                                          w.get(pre + "_residual_b"))


def _brute_forward(tokens, w, c, kv, known, position, group, role, covariates, rows, enc, h):
    n, d, heads, dh = enc + h, c.d_model, c.num_heads, c.head_dim
    ll = enc - h if covariates else enc
    emb = _res(tokens, w, "embed")
    x = np.zeros((rows * n, d))
    for i in range(rows):
        x[i * n: i * n + enc] = emb[i * enc: (i + 1) * enc]
        x[i * n + enc: (i + 1) * n] = w["query"]
    for lw in w["layers"]:
        for a in lw["attentions"]:
            hn = _rms(x, a["norm"], c.norm_eps)
            qkv = _lin(hn, a["qkv"]).astype(np.float32)
            if a["time"]:
                att = brute.ts_time(qkv, kv, known, position, rows, enc, ll, n, heads, dh, d, c.rope_dim, c.rope_theta)
            else:
                att = brute.ts_variate(qkv, kv, group, role, covariates, rows, enc, n, heads, dh, d)
            att = att.astype(np.float64)
            if a["gate"] is not None:
                att = att / (1.0 + np.exp(-_lin(hn, a["gate"])))
            x = x + _lin(att, a["wo"])
        hn = _rms(x, lw["mlp_norm"], c.norm_eps)
        f = lw["down"].shape[1]
        up = _lin(hn, lw["up"])
        x = x + _lin(_silu(up[:, :f]) * up[:, f:], lw["down"])
    y = _rms(x, w["out_norm"], c.norm_eps)
    dec = np.concatenate([y[i * n + enc: (i + 1) * n] for i in range(rows)])
    return _res(dec, w, "head")


@pytest.mark.parametrize("covariates", [False, True])
def test_forward_matches_brute_force(oracle, covariates):
    c = TINY
    rows, enc, h = 6, 5, 2
    ll = enc - h if covariates else enc
    kv, known, position = cases.ts_layout(3, rows, enc, ll, h, known_frac=0.4 if covariates else 0.0)
    group = np.array([0, 0, 0, 1, 1, 1], np.int32)
    role = np.array([0, 1, 2, 0, 1, 1] if covariates else [0] * rows, np.int32)
    w = tm.random_weights(c, seed=1, std=0.2)
    r = np.random.default_rng(2)
    tok = r.standard_normal((rows * enc, 2 * c.patch_size)).astype(np.float32)
    got = oracle.ts_forward_raw(tok, w, kv, known, position, group, role, covariates, rows, enc, ll, h, c.num_heads,
                                c.head_dim, c.rope_dim, c.norm_eps, c.rope_theta)
    exp = _brute_forward(tok, w, c, kv, known, position, group, role, covariates, rows, enc, h)
    assert got.shape == (rows * h, c.patch_size * c.num_quantiles)
    err = np.max(np.abs(got - exp)) / np.max(np.abs(exp))
    assert err < 2e-5, err


# ---- the host ends: BlockPrep.of / Quantiles.apply / BlockPrep.finish ---------------------------------

def test_prep_closed_forms(oracle):
    """A constant row: loc = the value, the causal std 0 floored at minimum_scale, so observed steps
    scale to 0; a binary known covariate: (0, 1) and no arcsinh; an unobserved step: 0 and a missing
    flag."""
    ps = 4
    window = np.array([[5.0] * 8, [0, 1, 1, 0, 1, 0, 0, 1], [1.0, 2, 3, 4, 5, 6, 7, 8]], np.float32)
    obs = np.ones((3, 8), bool)
    obs[2, 5] = False
    tok, scaled, loc, scale = oracle.ts_block_prep(window, obs, [0, 1, 0], ps, 1e-6, True)
    assert np.all(loc[0] == 5) and np.all(scale[0] == np.float32(1e-6)) and np.all(scaled[0] == 0)
    assert np.all(loc[1] == 0) and np.all(scale[1] == 1)
    np.testing.assert_array_equal(scaled[1], window[1])  # binary: (x - 0) / 1, no arcsinh
    # causal patch frames of a ramp: patch 0 mean 2.5, sample std sqrt(5/3)
    assert loc[2][0] == np.float32(2.5) and scale[2][0] == np.float32(np.sqrt(5.0 / 3.0))
    assert scaled[2][5] == 0 and tok[2 * 2 + 1][ps + 1] == 1 and tok[2 * 2 + 1][1] == 0
    assert scaled[2][0] == np.float32(np.arcsinh(np.float32((1.0 - 2.5) / np.float32(np.sqrt(5.0 / 3.0)))))


def test_quantile_map_closed_forms(oracle):
    """Zero raw deltas: softplus(0) = ln 2, so level i sits width_factor * ln 2 * (cumulative dp)
    from the median; large raw deltas pass through softplus as themselves."""
    knots = (0.1, 0.5, 0.9)
    raw = np.array([[0.0, 3.0, 0.0], [25.0, -1.0, 30.0]], np.float32)
    got = oracle.ts_quantile_map(raw, knots, 1, 2.0)
    w = np.float32(2.0) * np.float32(0.4)
    ln2 = np.float32(np.log1p(np.exp(0.0)))
    np.testing.assert_array_equal(got[0], [np.float32(3.0) - np.float32(w * ln2), 3.0, np.float32(3.0) + np.float32(w * ln2)])
    np.testing.assert_array_equal(got[1], [np.float32(-1.0) - np.float32(w * 25), -1.0, np.float32(-1.0) + np.float32(w * 30)])
    assert np.all(np.diff(got, axis=1) >= 0)


def _block(seed, rows, t, ps, nan_frac=0.1):
    r = np.random.default_rng(seed)
    x = (10 + 3 * r.standard_normal((rows, t))).astype(np.float32)
    obs = r.random((rows, t)) >= nan_frac
    obs[0, : ps + 1] = False
    return x, obs


@pytest.mark.parametrize("asinh", [True, False])
def test_host_prep_matches_oracle(oracle, asinh):
    c = tm.TimestralConfig(patch_size=4, use_asinh=asinh, quantiles=(0.1, 0.5, 0.9))
    x, obs = _block(3, 5, 24, 4)
    x[3] = (x[3] > 10).astype(np.float32)  # a binary row
    known = np.array([0, 0, 1, 1, 0])
    tok, scaled, loc, scale = tm.block_prep(c, x, obs, known)
    e_tok, e_scaled, e_loc, e_scale = oracle.ts_block_prep(x, obs, known, 4, c.minimum_scale, asinh)
    np.testing.assert_array_max_ulp(loc, e_loc, maxulp=1)
    np.testing.assert_array_max_ulp(scale, e_scale, maxulp=1)
    np.testing.assert_array_max_ulp(tok, e_tok, maxulp=2)
    np.testing.assert_array_max_ulp(scaled, e_scaled, maxulp=2)


def test_host_finish_matches_oracle(oracle):
    c = tm.TimestralConfig(patch_size=4, quantiles=(0.1, 0.2, 0.5, 0.8, 0.9))
    r = np.random.default_rng(4)
    rows, h, ll = 3, 2, 5
    raw = r.standard_normal((rows * h, 4 * 5)).astype(np.float32)
    raw[0, 2] = 89.0  # step 0's median: sinh(89) is finite, the levels above overflow and are clamped
    loc = (5 + r.standard_normal((rows, 6 * 4))).astype(np.float32)
    scale = np.abs(r.standard_normal((rows, 6 * 4))).astype(np.float32) + np.float32(0.1)
    got = tm.block_finish(c, raw, loc, scale, ll, h)
    exp = oracle.ts_block_finish(raw, loc, scale, ll, h, 4, c.quantiles, c.median_index, c.quantile_width_factor, True)
    assert np.all(np.isfinite(got))
    assert got[0, 0, 4] == got[0, 0, 2] > 1e37  # +inf clamped to the step's finite maximum
    np.testing.assert_array_max_ulp(got, exp, maxulp=2)


def _anchor_case(rows=3, ll=5, h=2, ps=4, extra_patches=0):
    """raw medians, and loc / scale that differ at every step of the window (so each step names a
    distinct frame)."""
    r = np.random.default_rng(8)
    w = (ll + extra_patches) * ps
    raw = r.uniform(-2, 2, (rows * h, ps)).astype(np.float32)
    loc = (100 * np.arange(rows * w).reshape(rows, w) + 3).astype(np.float32)
    scale = (1 + 0.01 * np.arange(rows * w).reshape(rows, w)).astype(np.float32)
    return raw, loc, scale, w


def _anchor_expected(raw, loc, scale, rows, ll, h, ps):
    """sinh(m) * scale[(ll-1)*P] + loc[(ll-1)*P] per step, float multiply then add."""
    a = (ll - 1) * ps
    m = np.sinh(raw.astype(np.float64)).astype(np.float32).reshape(rows, h * ps)
    return ((m * scale[:, a:a + 1]).astype(np.float32) + loc[:, a:a + 1]).astype(np.float32)


@pytest.mark.parametrize("extra", [0, 2])
def test_finish_anchor_closed_form(oracle, extra):
    """BlockPrep.finish denormalizes every forecast step with the frame at step (ll - 1) * P of the
    window, the first step of the last context patch (BlockPrep.java:91-95). With one (median) level
    the quantile map leaves the raw value, so each output is sinh(m) * scale[a] + loc[a] at that
    anchor; loc and scale differ at every step, so any other anchor fails. extra: a covariate
    window's horizon patches after the context (w = (ll + h) * P), which the anchor must skip."""
    rows, ll, h, ps = 3, 5, 2, 4
    raw, loc, scale, _ = _anchor_case(rows, ll, h, ps, extra)
    exp = _anchor_expected(raw, loc, scale, rows, ll, h, ps)
    got = oracle.ts_block_finish(raw, loc, scale, ll, h, ps, (0.5,), 0, 2.0, True)
    np.testing.assert_array_equal(got[:, :, 0], exp)
    c = tm.TimestralConfig(patch_size=ps, quantiles=(0.5,))
    np.testing.assert_array_equal(tm.block_finish(c, raw, loc, scale, ll, h)[:, :, 0], exp)
    # a wrong anchor is visible: the last step of the context, or (inside a covariate window) step ll * P
    for wrong in (ll * ps - 1, ll * ps)[: 1 + (extra > 0)]:
        assert not np.array_equal(exp, ((np.sinh(raw.astype(np.float64)).astype(np.float32).reshape(rows, -1)
                                         * scale[:, wrong:wrong + 1]) + loc[:, wrong:wrong + 1]).astype(np.float32))
