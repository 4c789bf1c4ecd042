"""GPU parity of the forecast's host ends on the device (jc_c2_prep: ModelLayout's cut and live mask
plus ModelPrep.of; jc_c2_finish: ModelPrep.finish) against the oracle's restatements (c2_prep,
c2_live, c2_finish, pinned in test_oracle_forward.py).

Bars: live exact; loc and scale within 2 float ulps (only the order of the double sums differs);
tokens and forecasts within 1e-6 by the reference's metric, with all but a handful of values
bit-identical (every operation rounds as the reference's does, no fused multiply-adds).
"""
import numpy as np
import pytest
import torch

from jitcast_amd import JitcastArgumentError, chronos2
from jitcast_amd import chronos2_model as cm
from jitcast_amd import rng

pytestmark = pytest.mark.gpu


def _series(seed, rows, t, lead_nan, gaps=0.0):
    x = rng.normal(rng.stream_seed(seed, 0), rows * t, 3.0).reshape(rows, t) + 10.0
    for i, k in enumerate(lead_nan):
        x[i, :k] = np.nan
    if gaps:
        hole = rng.uniform(rng.stream_seed(seed, 1), rows * t).reshape(rows, t) < gaps
        x[hole] = np.nan
    return x.astype(np.float32)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


CASES = [
    # rows, steps, context_length, patch, h, future steps, gaps, permuted
    (5, 200, 256, 16, 3, 20, 0.0, False),
    (6, 300, 256, 16, 2, 32, 0.2, True),   # cut to the last 256 steps
    (4, 37, 64, 16, 1, 0, 0.1, False),     # 37 steps: 11 NaN-padded leading values
    (3, 2048, 8192, 16, 4, 64, 0.0, True),
    (2, 16, 16, 16, 1, 5, 0.0, False),
]


@pytest.mark.parametrize("arcsinh", [True, False])
@pytest.mark.parametrize("rows,steps,cl,patch,h,fs,gaps,permuted", CASES)
def test_prep_matches_oracle(gpu, oracle, rows, steps, cl, patch, h, fs, gaps, permuted, arcsinh):
    print(f"case prep rows={rows} steps={steps} cl={cl} patch={patch} h={h} fs={fs} gaps={gaps} "
          f"permuted={permuted} arcsinh={arcsinh}", flush=True)
    lead = [0, steps, 7, steps // 2, 0, 3][:rows]
    x = _series(11 + rows, rows, steps, lead, gaps)
    if rows > 2:
        x[2, lead[2]:] = np.float32(4.5)  # a constant row: std 0, floored at 1e-5
    fut = None
    if fs:
        fut = np.full((rows, fs), np.nan, np.float32)
        fut[-1] = np.linspace(-2, 3, fs, dtype=np.float32)
    order = np.arange(rows, dtype=np.int32)[::-1].copy() if permuted else None
    c = cm.Chronos2Config(context_length=cl, patch_size=patch, time_encoding_scale=cl)
    lay = cm.layout(c, x[order] if permuted else x, np.zeros(rows, np.int32),
                    fut[order] if (permuted and fut is not None) else fut, h)
    tok_e, loc_e, scale_e = oracle.c2_prep(lay.window, lay.future, lay.nc, h, patch, c.time_encoding_scale, arcsinh)
    live_e = oracle.c2_live(lay.window, rows, lay.nc, patch, 1, h)
    tok, loc, scale, live, nc = chronos2.prep(_dev(x), _dev(fut) if fut is not None else None,
                                              _dev(order) if permuted else None, rows, cl, patch, h, 1,
                                              c.time_encoding_scale, arcsinh)
    torch.cuda.synchronize()
    assert nc == lay.nc
    np.testing.assert_array_equal(live.cpu().numpy().reshape(rows, -1), live_e.reshape(rows, -1))
    np.testing.assert_array_max_ulp(loc.cpu().numpy(), loc_e, maxulp=2)
    np.testing.assert_array_max_ulp(scale.cpu().numpy(), scale_e, maxulp=2)
    got = tok.cpu().numpy()
    err = oracle.rel_max_error(got, tok_e)
    same = float(np.mean(got == tok_e))
    print(f"  tokens rel err {err:.3e}, bit-identical {same:.6f}", flush=True)
    assert err <= 1e-6
    assert same >= 0.999


@pytest.mark.parametrize("arcsinh", [True, False])
@pytest.mark.parametrize("permuted", [False, True])
def test_finish_matches_oracle(gpu, oracle, arcsinh, permuted):
    rows, h, q, patch = 7, 3, 21, 16
    raw = rng.normal(rng.stream_seed(5, 0), rows * h * q * patch, 1.5).astype(np.float32).reshape(rows * h, q * patch)
    loc = rng.normal(rng.stream_seed(5, 1), rows, 5.0).astype(np.float32)
    scale = np.abs(rng.normal(rng.stream_seed(5, 2), rows, 2.0)).astype(np.float32) + np.float32(1e-3)
    order = np.random.default_rng(5).permutation(rows).astype(np.int32) if permuted else None
    exp = oracle.c2_finish(raw, loc, scale, rows, h, q, patch, arcsinh)
    if permuted:
        back = np.empty_like(exp)
        back[order] = exp
        exp = back
    out = torch.empty(rows, q, h * patch, dtype=torch.float32, device="cuda")
    chronos2.finish(_dev(raw), _dev(loc), _dev(scale), _dev(order) if permuted else None, rows, h, q, patch, arcsinh,
                    out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    err = oracle.rel_max_error(got, exp)
    same = float(np.mean(got == exp))
    print(f"finish arcsinh={arcsinh} permuted={permuted}: rel err {err:.3e}, bit-identical {same:.6f}", flush=True)
    assert err <= 1e-6
    assert same >= 0.999


def test_forecast_rejects_bad_arguments(gpu):
    c = cm.Chronos2Config(d_model=64, d_kv=16, d_ff=128, num_layers=1, num_heads=4, context_length=64,
                          quantiles=(0.5,), time_encoding_scale=64)
    m = cm.HipChronos2Model(c, cm.random_weights(c, seed=0))
    x = np.zeros((2, 40), np.float32)
    with pytest.raises(JitcastArgumentError):
        m.forecast(x, [0, 1], h=0)
    with pytest.raises(JitcastArgumentError):
        m.forecast(x, [0], h=1)
    with pytest.raises(JitcastArgumentError):
        m.forecast(x, [0, 1], np.zeros((2, 40), np.float32), h=2)
