"""GPU parity of the Timestral block's host ends on the device: jc_ts_prep (BlockPrep.of,
J/timestral/BlockPrep.java:40-75, with Scaler.causalPatchLocScale / instanceNorm / affine) and
jc_ts_finish (BlockPrep.finish, BlockPrep.java:77-101, with Quantiles.apply and
Scaler.invert / clampNonFinite) against the oracle's value-by-value restatements (pinned in
test_oracle_ts_forward.py). The running double sums keep the reference's step order, so loc, scale
and the flags match exactly; values that pass through a double log / sqrt / exp / sinh of the
device's math library are within one float ulp; NaN lands where the reference's NaN lands."""
import numpy as np
import pytest
import torch

from jitcast_amd import _lib, chronos2
from jitcast_amd import timestral_model as tm

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ulps(a, b):
    """Largest distance in float ulps between a and b, with NaN required at the same places."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb), f"NaN at {np.argwhere(na != nb)[:5].tolist()}"
    a, b = a[~na], b[~nb]
    if a.size == 0:
        return 0
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)  # ordered integer line through -0 / +0
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return int(np.max(np.abs(ia - ib)))


def _prep(window, observed, known, patch, minimum_scale, use_asinh):
    rows, w = window.shape
    enc = w // patch
    win = torch.from_numpy(np.ascontiguousarray(window, np.float32)).to(DEV)
    obs = torch.from_numpy(np.ascontiguousarray(observed, np.uint8)).to(DEV)
    kn = torch.from_numpy(np.ascontiguousarray(known, np.int32)).to(DEV)
    tok = torch.full((rows * enc, 2 * patch), 7.0, device=DEV)
    scaled = torch.full((rows, w), 7.0, device=DEV)
    loc = torch.full((rows, w), 7.0, device=DEV)
    scale = torch.full((rows, w), 7.0, device=DEV)
    p = chronos2._ptr
    _lib.call("jc_ts_prep", chronos2.context(0).handle, p(win), p(obs), rows, w, patch, p(kn), minimum_scale,
              int(use_asinh), p(tok), p(scaled), p(loc), p(scale))
    torch.cuda.synchronize()
    return tok.cpu().numpy(), scaled.cpu().numpy(), loc.cpu().numpy(), scale.cpu().numpy()


def _series(r, rows, w):
    x = (50 + 10 * np.sin(np.arange(w) / 7.0)[None, :] + 3 * r.standard_normal((rows, w))).astype(np.float32)
    obs = r.random((rows, w)) > 0.15
    return x, obs


# (name, rows, patch, enc): patch 16 (4 patches per 64-lane chunk), 24 (2 per chunk, lanes 48..63
# idle), 5 (12 per chunk), 64 (one per chunk), 1
PREP_CASES = [("p16", 5, 16, 37), ("p24", 4, 24, 11), ("p5", 3, 5, 50), ("p64", 3, 64, 6), ("p1", 2, 1, 150)]


@pytest.mark.parametrize("name,rows,patch,enc", PREP_CASES, ids=[c[0] for c in PREP_CASES])
@pytest.mark.parametrize("use_asinh", [True, False])
def test_prep_causal_matches_oracle(gpu, oracle, name, rows, patch, enc, use_asinh):
    print(f"case ts_prep causal {name} asinh={use_asinh}", flush=True)
    r = np.random.default_rng(31 + patch)
    w = enc * patch
    x, obs = _series(r, rows, w)
    obs[0, : 3 * patch + 1] = False  # leading unobserved patches: mean 0, scale at the floor
    if rows > 2:
        obs[2] = False  # nothing observed at all
    known = np.zeros(rows, np.int32)
    got = _prep(x, obs, known, patch, 1e-6, use_asinh)
    exp = oracle.ts_block_prep(x, obs, known, patch, 1e-6, use_asinh)
    tok, scaled, loc, scale = got
    np.testing.assert_array_equal(loc, exp[2])
    assert _ulps(scale, exp[3]) <= 1
    assert _ulps(scaled, exp[1]) <= 1
    assert _ulps(tok, exp[0]) <= 1
    np.testing.assert_array_equal(tok[:, patch:], exp[0][:, patch:])  # missing flags exactly


def test_prep_known_rows_match_oracle(gpu, oracle):
    """Known covariate rows take the whole-row instance norm; a 0/1 row is binary (loc 0, scale 1,
    no arcsinh); a row with nothing observed keeps the scale floor; other rows stay causal."""
    print("case ts_prep known rows", flush=True)
    r = np.random.default_rng(41)
    rows, patch, enc = 6, 16, 20
    w = enc * patch
    x, obs = _series(r, rows, w)
    x[1] = (r.random(w) > 0.5).astype(np.float32)  # an indicator covariate
    x[1, ~obs[1]] = 5.0  # values at unobserved steps do not break the 0/1 test
    obs[3] = False
    x[4] = 1e4 + r.standard_normal(w).astype(np.float32) * 1e-2  # near-constant: order-sensitive sums
    known = np.array([0, 1, 1, 1, 1, 0], np.int32)
    for use_asinh in (True, False):
        got = _prep(x, obs, known, patch, 1e-6, use_asinh)
        exp = oracle.ts_block_prep(x, obs, known, patch, 1e-6, use_asinh)
        np.testing.assert_array_equal(got[2], exp[2])
        np.testing.assert_array_equal(got[3], exp[3])
        assert _ulps(got[1], exp[1]) <= 1
        assert _ulps(got[0], exp[0]) <= 1
    assert got[2][1, 0] == 0.0 and got[3][1, 0] == 1.0


def test_prep_nan_propagates_as_reference(gpu, oracle):
    """A NaN value at a missing step still enters the reference's running sums (0 * NaN): loc and
    scale turn NaN from that step's patch on, as the reference's do."""
    print("case ts_prep NaN", flush=True)
    r = np.random.default_rng(43)
    rows, patch, enc = 3, 16, 12
    w = enc * patch
    x, obs = _series(r, rows, w)
    obs[0, 100] = False
    x[0, 100] = np.nan
    known = np.array([0, 0, 1], np.int32)
    obs[2, 7] = False
    x[2, 7] = np.nan
    got = _prep(x, obs, known, patch, 1e-6, True)
    exp = oracle.ts_block_prep(x, obs, known, patch, 1e-6, True)
    for g, e in zip(got, exp):
        assert _ulps(g, e) <= 1
    assert np.isnan(got[2][0, 96]) and not np.isnan(got[2][0, 95])


def test_prep_config3_shape_properties(gpu, oracle):
    """At config 3's row length (1023 patches of 16, left padding) the oracle's loops are too slow
    for many rows; check two rows against it and the rest by properties: the first observed patch's
    loc is its own mean, flags are exact, tokens are the scaled window."""
    print("case ts_prep config-3 rows", flush=True)
    r = np.random.default_rng(47)
    rows, patch, enc = 16, 16, 1023
    w = enc * patch
    x = r.standard_normal((rows, w)).astype(np.float32)
    pad = r.integers(0, 257, rows)
    obs = np.arange(w)[None, :] >= (pad * patch)[:, None]
    known = np.zeros(rows, np.int32)
    tok, scaled, loc, scale = _prep(x, obs, known, patch, 1e-6, True)
    exp = oracle.ts_block_prep(x[:2], obs[:2], known[:2], patch, 1e-6, True)
    np.testing.assert_array_equal(loc[:2], exp[2])
    assert _ulps(scale[:2], exp[3]) <= 1
    assert _ulps(scaled[:2], exp[1]) <= 1
    for i in range(rows):
        s = pad[i] * patch
        assert np.all(loc[i, :s] == 0) and np.all(scale[i, :s] == np.float32(1e-6))
        m = np.float32(np.mean(x[i, s:s + patch].astype(np.float64)))
        assert abs(loc[i, s] - m) <= 1e-6 * max(1.0, abs(m))
    t3 = tok.reshape(rows, enc, 2 * patch)
    np.testing.assert_array_equal(t3[:, :, :patch].reshape(rows, w), scaled)
    np.testing.assert_array_equal(t3[:, :, patch:].reshape(rows, w), (~obs).astype(np.float32))


@pytest.mark.parametrize("quantiles,use_asinh", [((0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9), True),
                                                 ((0.1, 0.5, 0.9), False), ((0.25, 0.5, 0.75, 0.95), True)])
def test_finish_matches_oracle(gpu, oracle, quantiles, use_asinh):
    print(f"case ts_finish q={len(quantiles)} asinh={use_asinh}", flush=True)
    c = tm.TimestralConfig(patch_size=8, quantiles=quantiles, use_asinh=use_asinh)
    r = np.random.default_rng(53)
    rows, ll, h, ps, q = 5, 9, 3, 8, len(quantiles)
    w = ll * ps
    loc = (10 * r.standard_normal((rows, w))).astype(np.float32)
    scale = np.abs(r.standard_normal((rows, w))).astype(np.float32) + 0.1
    raw = (2 * r.standard_normal((rows * h, ps * q))).astype(np.float32)
    raw[0, :q] = 25.0  # softplus's identity branch
    raw[1, :q] = [200.0] * q  # sinh overflows to inf: clamped to the finite extremes or 0
    raw[2, 0] = -200.0
    exp = oracle.ts_block_finish(raw, loc, scale, ll, h, ps, quantiles, c.median_index, c.quantile_width_factor,
                                 use_asinh)
    p = chronos2._ptr
    widths = tm.quantile_widths(c)
    loc_d, scale_d = torch.from_numpy(loc).to(DEV), torch.from_numpy(scale).to(DEV)  # held until the kernel ran
    for in_place in (False, True):
        rd = torch.from_numpy(raw.copy()).to(DEV)
        out = rd if in_place else torch.full((rows, h * ps, q), 7.0, device=DEV)
        _lib.call("jc_ts_finish", chronos2.context(0).handle, p(rd), p(loc_d), p(scale_d), rows, w, ll, h, ps, q,
                  widths.ctypes.data, c.median_index, int(use_asinh), p(out))
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(rows, h * ps, q)
        assert _ulps(got, exp) <= 1
        assert np.all(np.isfinite(got))
        assert np.all(np.diff(got, axis=2) >= 0)


def test_ends_reject_bad_arguments(gpu):
    ctx = chronos2.context(0)
    a = torch.zeros(64, device=DEV)
    p = chronos2._ptr(a)
    with pytest.raises(_lib.JitcastError, match="patch"):
        _lib.call("jc_ts_prep", ctx.handle, p, p, 1, 48, 80, None, 1e-6, 1, p, None, p, p)
    with pytest.raises(_lib.JitcastError, match="patch"):
        _lib.call("jc_ts_prep", ctx.handle, p, p, 1, 50, 16, None, 1e-6, 1, p, None, p, p)
    w = np.ones(40, np.float32)
    with pytest.raises(_lib.JitcastError, match="q <= 32"):
        _lib.call("jc_ts_finish", ctx.handle, p, p, p, 1, 16, 1, 1, 16, 40, w.ctypes.data, 20, 1, p)
    with pytest.raises(_lib.JitcastError, match="exceeds the window"):
        _lib.call("jc_ts_finish", ctx.handle, p, p, p, 1, 16, 2, 1, 16, 3, w.ctypes.data, 1, 1, p)


@pytest.mark.parametrize("extra", [0, 2])
def test_finish_anchor_closed_form(gpu, extra):
    """jc_ts_finish's frame is the window's step (ll - 1) * P (BlockPrep.java:91-95): with loc and
    scale different at every step and one (median) level, each output is sinh(m) * scale[a] + loc[a]
    (tests/test_oracle_ts_forward.py pins the same closed form on the oracle)."""
    from tests.test_oracle_ts_forward import _anchor_case, _anchor_expected

    rows, ll, h, ps = 3, 5, 2, 4
    raw, loc, scale, w = _anchor_case(rows, ll, h, ps, extra)
    exp = _anchor_expected(raw, loc, scale, rows, ll, h, ps)
    widths = np.zeros(1, np.float32)
    p = chronos2._ptr
    rd, loc_d, scale_d = (torch.from_numpy(a).to(DEV) for a in (raw, loc, scale))
    out = torch.empty(rows, h * ps, 1, device=DEV)
    _lib.call("jc_ts_finish", chronos2.context(0).handle, p(rd), p(loc_d), p(scale_d), rows, w, ll, h, ps, 1,
              widths.ctypes.data, 0, 1, p(out))
    torch.cuda.synchronize()
    got = out.cpu().numpy()[:, :, 0]
    assert _ulps(got, exp) <= 1  # the device's sinh may differ from the host's by one ulp
