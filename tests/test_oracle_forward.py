"""Pins of the oracle's Chronos-2 forward pieces (ModelPrep.of / instanceNorm / finish, J/chronos2/
ModelPrep.java:38-151; CpuChronos2.forward, J/chronos2/cpu/CpuChronos2.java:122-169) against
closed forms and float64 restatements, and of the host mirror's ModelLayout / ModelPrep / finish
(jitcast_amd.chronos2_model) against the oracle. CPU only."""
import numpy as np
import pytest

from jitcast_amd import chronos2_model as cm
from tests.test_oracle_ops import _brute_layer

pytestmark = pytest.mark.usefixtures("oracle")

TINY = cm.Chronos2Config(d_model=32, d_kv=8, d_ff=48, num_layers=2, num_heads=2, context_length=64, patch_size=4,
                         quantiles=(0.1, 0.5, 0.9), time_encoding_scale=64)


def _context(seed, rows, t, nan_frac=0.2, lead_nan=None):
    r = np.random.default_rng(seed)
    x = (3 + 2 * r.standard_normal((rows, t))).astype(np.float32)
    x[r.random((rows, t)) < nan_frac] = np.nan
    if lead_nan is not None:
        for i, k in enumerate(lead_nan):
            x[i, :k] = np.nan
    return x


def _ulps(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.max(np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))) if a.size else 0


def test_instance_norm_closed_form(oracle):
    x = _context(1, 5, 37)
    x[3] = np.nan  # no observation: (0, 1)
    x[4] = 2.5  # constant: std floored at 1e-5
    for i in range(5):
        loc, scale = oracle.c2_instance_norm(x[i])
        obs = x[i][~np.isnan(x[i])]
        if obs.size == 0:
            assert (loc, scale) == (0.0, 1.0)
            continue
        m = np.float32(obs.astype(np.float64).mean())
        sd = np.float32(np.sqrt(((obs - m).astype(np.float32).astype(np.float64) ** 2).mean()))
        assert loc == m
        assert scale == (np.float32(1e-5) if sd == 0 else sd)


@pytest.mark.parametrize("arcsinh", [False, True])
def test_prep_tokens_and_finish(oracle, arcsinh):
    nc, h, ps, ts = 3, 2, 4, 64
    win = _context(2, 2, nc * ps)
    fut = np.full((2, h * ps), np.nan, np.float32)
    fut[1, :5] = [0.5, -1.0, 2.0, 0.0, 7.0]
    tok, loc, scale = oracle.c2_prep(win, fut, nc, h, ps, ts, arcsinh)
    tok = tok.reshape(2, nc + h, 3 * ps)
    # time encoding: context steps count up to -1 / ts, future steps from 0
    np.testing.assert_array_equal(tok[0, :nc, :ps].reshape(-1), ((np.arange(nc * ps) - nc * ps) / np.float32(ts)).astype(np.float32))
    np.testing.assert_array_equal(tok[0, nc:, :ps].reshape(-1), (np.arange(h * ps) / np.float32(ts)).astype(np.float32))
    # masks and values
    obs = ~np.isnan(win)
    np.testing.assert_array_equal(tok[:, :nc, 2 * ps:].reshape(2, -1), obs.astype(np.float32))
    z = (win.astype(np.float64) - loc[:, None]) / scale[:, None]
    expect = np.arcsinh(z) if arcsinh else z
    got = tok[:, :nc, ps:2 * ps].reshape(2, -1)
    np.testing.assert_allclose(got[obs], expect[obs], rtol=2e-6, atol=1e-6)
    assert (got[~obs] == 0).all()
    assert tok[1, nc, 2 * ps:].tolist() == [1, 1, 1, 1] and tok[1, nc + 1, 2 * ps:].tolist() == [1, 0, 0, 0]
    # finish inverts the scaling: raw = scaled(x) gives back x
    raw = np.zeros((2 * h, 3 * ps), np.float32)
    raw[:, ps:2 * ps] = 0.75
    out = oracle.c2_finish(raw, loc, scale, 2, h, 3, ps, arcsinh)
    v = np.sinh(0.75) if arcsinh else 0.75
    np.testing.assert_allclose(out[:, 1, :], (v * scale[:, None] + loc[:, None]) * np.ones((2, h * ps)), rtol=1e-6)
    np.testing.assert_allclose(out[:, 0, :], loc[:, None] * np.ones((2, h * ps)), rtol=1e-6)


def test_host_layout_rules(oracle):
    c = TINY
    ctx = _context(3, 3, 70, lead_nan=[0, 30, 70])  # longer than context_length (64): cut to the last 64
    fc = np.arange(6, dtype=np.float32).reshape(3, 2)
    lay = cm.layout(c, ctx, [0, 1, 1], fc, h=2)
    assert (lay.nc, lay.nreg, lay.h, lay.n) == (16, 1, 2, 19)
    np.testing.assert_array_equal(lay.window[:, :], ctx[:, 6:])
    assert np.isnan(lay.future[:, 2:]).all() and (lay.future[:, :2] == fc).all()
    # live: a context patch with an observed value; [REG] and future always
    exp = np.ones((3, 19), np.int32)
    for i in range(3):
        for p in range(16):
            exp[i, p] = int(not np.isnan(lay.window[i, 4 * p: 4 * p + 4]).all())
    np.testing.assert_array_equal(lay.live, exp)
    assert lay.live[2, :16].sum() == 0  # the row with no observation at all
    with pytest.raises(ValueError):
        cm.layout(c, ctx, [0, 1, 1], np.zeros((3, 9), np.float32), h=2)  # 9 future steps > 2 patches
    with pytest.raises(ValueError):
        cm.layout(c, ctx, [0, 1], None, h=2)
    # short context: padded on the left to whole patches
    lay = cm.layout(c, ctx[:, :10], [0, 0, 0], None, h=1)
    assert lay.nc == 3 and np.isnan(lay.window[:, :2]).all()


@pytest.mark.parametrize("arcsinh", [False, True])
def test_host_prep_and_finish_match_oracle(oracle, arcsinh):
    c = cm.Chronos2Config(**{**TINY.__dict__, "use_arcsinh": arcsinh})
    ctx = _context(4, 4, 45, lead_nan=[0, 5, 45, 12])
    ctx[0, 7] = 1e6  # an outlier
    lay = cm.layout(c, ctx, [0, 0, 1, 1], np.full((4, 3), 0.25, np.float32), h=2)
    tok, loc, scale = cm.prep(c, lay)
    otok, oloc, oscale = oracle.c2_prep(lay.window, lay.future, lay.nc, lay.h, c.patch_size, c.time_encoding_scale,
                                        arcsinh)
    # the sums run in a different order (pairwise against sequential): at most one float ulp apart
    assert _ulps(loc, oloc) <= 1 and _ulps(scale, oscale) <= 1
    assert _ulps(tok, otok) <= 2
    raw = np.random.default_rng(5).standard_normal((4 * 2, c.num_quantiles * c.patch_size)).astype(np.float32)
    assert _ulps(cm.finish(c, lay, raw, oloc, oscale),
                 oracle.c2_finish(raw, oloc, oscale, 4, 2, c.num_quantiles, c.patch_size, arcsinh)) <= 1


def _brute_forward(tokens, w, live, group, rows, nc, nreg, h, heads, dh, eps):
    """float64: residual blocks, token order, layers (_brute_layer), final norm, future tokens."""
    def lin(v, wk, bk):
        return v @ w[wk].astype(np.float64).T + w[bk].astype(np.float64)

    def res(v, pre):
        hid = np.maximum(lin(v, pre + "_hidden_w", pre + "_hidden_b"), 0)
        return lin(hid, pre + "_output_w", pre + "_output_b") + lin(v, pre + "_residual_w", pre + "_residual_b")

    ne, n = nc + h, nc + nreg + h
    emb = res(tokens.astype(np.float64), "in")
    x = []
    for i in range(rows):
        parts = [emb[i * ne: i * ne + nc]]
        if nreg:
            parts.append(w["shared"][1:2].astype(np.float64))
        parts.append(emb[i * ne + nc: (i + 1) * ne])
        x.append(np.concatenate(parts))
    x = np.concatenate(x)
    for lw in w["layers"]:
        x = _brute_layer(x, lw, live, group, rows, n, heads, dh, eps)
    y = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w["final_norm"].astype(np.float64)
    dec = np.concatenate([y[i * n + nc + nreg: (i + 1) * n] for i in range(rows)])
    return res(dec, "out")


def test_forward_composition_matches_brute_force(oracle):
    c = TINY
    w = cm.random_weights(c, seed=6, std=0.2)
    ctx = _context(7, 4, 30, lead_nan=[0, 6, 0, 13])
    lay = cm.layout(c, ctx, [0, 0, 1, 1], None, h=2)
    tok, _, _ = oracle.c2_prep(lay.window, lay.future, lay.nc, lay.h, c.patch_size, c.time_encoding_scale, True)
    got = oracle.c2_forward_raw(tok, w, lay.live, lay.group, lay.rows, lay.nc, lay.nreg, lay.h, c.num_heads, c.d_kv,
                                c.layer_norm_eps)
    exp = _brute_forward(tok, w, lay.live, lay.group, lay.rows, lay.nc, lay.nreg, lay.h, c.num_heads, c.d_kv,
                         c.layer_norm_eps)
    assert got.shape == (4 * 2, c.num_quantiles * c.patch_size)
    assert oracle.rel_max_error(got, exp) <= 1e-5
