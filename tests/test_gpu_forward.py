"""GPU parity of the Chronos-2 forward (jitcast_amd.chronos2_model.HipChronos2Model: the input patch
embedding, token assembly, encoder layers, final norm, future gather and output patch embedding on
the device through the C ABI) against the oracle's CpuChronos2.forward restatement.

Bars: the raw output patch embedding within 1e-4 (fp32); the quantile forecasts within 1e-3 (the
end-to-end bar); a bf16 encoder within 2e-2.
"""
import numpy as np
import pytest
import torch

from jitcast_amd import chronos2_model as cm
from tests.test_oracle_forward import _context

pytestmark = pytest.mark.gpu

SMALL = cm.Chronos2Config(d_model=64, d_kv=16, d_ff=128, num_layers=2, num_heads=4, context_length=256, patch_size=16,
                          quantiles=(0.1, 0.5, 0.9), time_encoding_scale=256)
# config 0's model: Chronos-2 28M-class (d_model 512, 8 x 64, 6 layers, patch 16), 21 quantiles
CONFIG0 = cm.Chronos2Config(d_model=512, d_kv=64, d_ff=2048, num_layers=6, num_heads=8)


def _oracle_forecast(oracle, c, w, lay):
    tok, loc, scale = oracle.c2_prep(lay.window, lay.future, lay.nc, lay.h, c.patch_size, c.time_encoding_scale,
                                     c.use_arcsinh)
    raw = oracle.c2_forward_raw(tok, w, lay.live, lay.group, lay.rows, lay.nc, lay.nreg, lay.h, c.num_heads, c.d_kv,
                                c.layer_norm_eps, c.rope_theta)
    return tok, raw, oracle.c2_finish(raw, loc, scale, lay.rows, lay.h, c.num_quantiles, c.patch_size, c.use_arcsinh)


def test_forward_raw_matches_oracle(gpu, oracle):
    c = SMALL
    w = cm.random_weights(c, seed=1, std=0.1)
    lay = cm.layout(c, _context(2, 6, 200, lead_nan=[0, 40, 0, 200, 17, 0]), [0, 0, 1, 1, 1, 2], None, h=3)
    tok, raw, _ = _oracle_forecast(oracle, c, w, lay)
    m = cm.HipChronos2Model(c, w)
    dev = m.dev
    gs, ge = cm.chronos2.group_bounds(lay.group)
    got = m.forward_raw(torch.from_numpy(tok).to(dev), torch.from_numpy(lay.live.reshape(-1)).to(dev),
                        torch.from_numpy(gs).to(dev), torch.from_numpy(ge).to(dev), lay.rows, lay.nc, lay.h)
    torch.cuda.synchronize()
    err = oracle.rel_max_error(got.cpu().numpy(), raw)
    print(f"raw rel err {err:.3e}", flush=True)
    assert err <= 1e-4


@pytest.mark.parametrize("cfg", ["small", "config0"])
def test_forecast_matches_oracle(gpu, oracle, cfg):
    """End to end: layout, prep, device forward, finish; rows of a group not adjacent (the engine
    orders them and puts the forecasts back), one row with a known future covariate."""
    c = SMALL if cfg == "small" else CONFIG0
    w = cm.random_weights(c, seed=3, std=0.02 if cfg == "config0" else 0.1)
    rows = 5 if cfg == "small" else 4
    ctx = _context(4, rows, 512 if cfg == "config0" else 150, lead_nan=[0, 9, 0, 33, 0][:rows])
    group = [1, 0, 1, 0, 2][:rows]
    fc = np.zeros((rows, 20), np.float32)
    fc[:] = np.nan
    fc[rows - 1] = np.linspace(-1, 1, 20)
    h = 4 if cfg == "config0" else 2
    m = cm.HipChronos2Model(c, w)
    got = m.forecast(ctx, group, fc, h=h)
    # the oracle on the same rows in group order, mapped back
    lay = cm.layout(c, ctx, group, fc, h=h)
    order = np.argsort(np.asarray(group), kind="stable")
    lay_o = cm.Layout(lay.rows, lay.nc, lay.nreg, lay.h, lay.window[order], lay.future[order], lay.live[order],
                      lay.group[order])
    _, _, exp_o = _oracle_forecast(oracle, c, w, lay_o)
    exp = np.empty_like(exp_o)
    exp[order] = exp_o
    err = oracle.rel_max_error(got, exp)
    print(f"{cfg} forecast rel err {err:.3e}", flush=True)
    assert got.shape == (rows, c.num_quantiles, h * c.patch_size)
    assert err <= 1e-3


@pytest.mark.parametrize("dt", ["bf16", "fp16", "f16x3"])
def test_forecast_lowp_encoder(gpu, oracle, dt):
    """The encoder's other GEMM types on config 0's model: bf16 and fp16 within 2e-2, f16x3 (three-term
    fp16 splits, fp32 results) within the fp32 bar of 1e-3."""
    c = CONFIG0
    w = cm.random_weights(c, seed=5)
    ctx = _context(6, 3, 512, lead_nan=[0, 100, 7])
    m = cm.HipChronos2Model(c, w, dtype=dt)
    got = m.forecast(ctx, [0, 0, 1], None, h=2)
    lay = cm.layout(c, ctx, [0, 0, 1], None, h=2)
    _, _, exp = _oracle_forecast(oracle, c, w, lay)
    err = oracle.rel_max_error(got, exp)
    print(f"{dt} encoder forecast rel err {err:.3e}", flush=True)
    assert err <= (1e-3 if dt == "f16x3" else 2e-2)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16x3"])
def test_planned_forecast_matches_eager(gpu, dt):
    """HipChronos2Model with max_plans: the device forward captured once per
    Shape(rows, contextPatches, outputPatches) and replayed (Chronos2Forward.java:106, PlanCache.run).
    Every replay, with fresh inputs and eager work between replays, equals the eager forecast bit for
    bit; a third shape evicts the least recently used plan; the weights are not part of any plan's
    bytes."""
    print(f"case planned forecast {dt}", flush=True)
    c = SMALL
    w = cm.random_weights(c, seed=3, std=0.1)
    eager = cm.HipChronos2Model(c, w, dtype=dt)
    planned = cm.HipChronos2Model(c, w, dtype=dt, max_plans=2)
    try:
        # (rows, steps, groups, h): three shapes, the first one again after the second
        runs = [(6, 200, [0, 0, 1, 1, 1, 2], 2), (4, 96, [0, 1, 1, 2], 1), (6, 200, [0, 1, 1, 2, 2, 2], 2),
                (3, 256, [0, 0, 0], 3), (6, 200, [2, 2, 1, 0, 0, 1], 2)]
        for k, (rows, steps, group, h) in enumerate(runs):
            ctx = _context(10 + k, rows, steps, lead_nan=[(17 * k + 5 * i) % steps for i in range(rows)])
            got = planned.forecast(ctx, group, None, h=h)
            exp = eager.forecast(ctx, group, None, h=h)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(got, exp)
        nc = lambda steps: (min(steps, c.context_length) + c.patch_size - 1) // c.patch_size  # noqa: E731
        # shapes A = (6, 200, 2), B = (4, 96, 1), C = (3, 256, 3): A, B, A (hit), C evicts B, A (hit)
        assert planned.plans.keys() == [(3, nc(256), 3), (6, nc(200), 2)]
        weights = sum(t.numel() * t.element_size() for t in planned.w.values())
        assert 0 < planned.plans.cached_bytes() < 2 * weights + (64 << 20)
    finally:
        planned.close()
    assert planned.plans.keys() == []
