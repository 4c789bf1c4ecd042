"""GPU parity of the HIP Chronos-2 engine (jitcast_amd.engine.HipChronos2Engine: a checkpoint loaded from
config.json + model.safetensors, the host pipeline, the device forward) against the oracle: the
oracle's scalar restatement of Chronos2Pipeline over the oracle's CpuChronos2.forward.

The batch is the reference's mixed batch (Chronos2BatchParityAccelTest.java:45-115): ragged lengths,
late starts, gaps, bivariate targets, past-only and known covariates, four patches per pass so a
horizon of 100 unrolls once; every forward call is checked within 1e-4 (fp32) as that test does,
and the forecasts within 1e-3. The bf16 encoder's calls are held to 2e-2; its forecasts, where the
unrolled pass feeds rounded forecasts back in, to the reference's bar for its reduced-precision GEMM
modes on this batch, 5e-2 (REDUCED_TOLERANCE, Chronos2BatchParityAccelTest.java:42, 50).
"""
import numpy as np
import pytest

from jitcast_amd import checkpoint as ck
from jitcast_amd.api import TimeSeries
from jitcast_amd.chronos2_model import QUANTILES_21, Chronos2Config, random_weights
from jitcast_amd.engine import HipChronos2Engine
from oracle import c2_pipeline as ref
from tests.test_pipeline import _mixed_batch

pytestmark = pytest.mark.gpu

C = Chronos2Config(d_model=64, d_kv=16, d_ff=128, num_layers=2, num_heads=4, context_length=256, patch_size=16,
                   max_output_patches=4, quantiles=QUANTILES_21, time_encoding_scale=256)


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    d = tmp_path_factory.mktemp("c2ckpt")
    ck.write_chronos2(d, C, random_weights(C, seed=21, std=0.1))
    return d


def _oracle_forward(oracle, c, w):
    def fwd(context, group, future, op):
        return oracle.c2_model_forward(c, w, np.asarray(context, np.float32), np.asarray(group, np.int32),
                                       np.asarray(future, np.float32), op)
    return fwd


@pytest.mark.parametrize("dt,call_bar,bar", [("f32", 1e-4, 1e-3), ("f16x3", 1e-4, 1e-3), ("bf16", 2e-2, 5e-2)])
def test_engine_mixed_batch_matches_oracle_pipeline(gpu, oracle, checkpoint, dt, call_bar, bar):
    print(f"case engine mixed batch {dt}", flush=True)
    horizon = 100
    series = _mixed_batch(11, 25, horizon)
    _, w = ck.load_chronos2(checkpoint)
    calls = []
    with HipChronos2Engine.load(checkpoint, dtype=dt) as eng:
        fwd = eng.forward_pass()
        ofwd = _oracle_forward(oracle, C, w)

        def checked(inp):
            out = fwd(inp)
            exp = ofwd(inp.context, inp.group, inp.future_covariates, inp.output_patches)
            err = oracle.rel_max_error(out, exp)
            calls.append(err)
            print(f"  call{len(calls) - 1} rows={inp.rows()} length={inp.length()} patches={inp.output_patches} "
                  f"rel err {err:.2e}", flush=True)
            return out

        pipe = eng.pipeline()
        pipe.forward = checked
        got = pipe.forecast([TimeSeries(t, p, k) for t, p, k in series], horizon)
    exp = ref.forecast(C, _oracle_forward(oracle, C, w), series, horizon)
    assert len(calls) == 2, "the horizon unrolls once"
    assert max(calls) <= call_bar
    err = max(oracle.rel_max_error(g.values, e) for g, e in zip(got, exp))
    print(f"  forecasts rel err {err:.2e} (bar {bar:.0e})", flush=True)
    assert err <= bar


def test_engine_contract(gpu, checkpoint):
    """ForecastEngine's contract: a name, horizon checked, one Forecast per series in order with the
    model's levels, close() idempotent and final."""
    eng = HipChronos2Engine.load(checkpoint)
    assert eng.name() == "chronos2-hip"
    # plans on by default, as the reference's <model>.tornado.plans (8, docs/CONFIGURATION.md:56)
    assert eng.forward_pass().model.plans.max_plans == 8
    assert eng.config() == C
    s = [TimeSeries.univariate(np.sin(np.arange(200, dtype=np.float32) / 5)),
         TimeSeries([np.ones(90), np.arange(90)], None, [np.linspace(0, 1, 90 + 20)])]
    with pytest.raises(ValueError):
        eng.forecast(s, 0)
    out = eng.forecast(s, 20)
    assert [f.values.shape for f in out] == [(1, 21, 20), (2, 21, 20)]
    np.testing.assert_array_equal(out[0].levels, C.quantile_levels())
    assert np.isfinite(out[1].median(1)).all()
    # the same series alone gives the same forecast (no cross-learning): the batch does not leak
    alone = eng.forecast(s[:1], 20)
    np.testing.assert_allclose(alone[0].values, out[0].values, rtol=0, atol=1e-5)
    eng.close()
    eng.close()
    with pytest.raises(RuntimeError):
        eng.forecast(s, 20)


def test_config0_fixture_through_the_engine(gpu, oracle, tmp_path):
    """Config 0 end to end on the GPU against the committed oracle fixture: the 28M-class checkpoint
    written as config.json + model.safetensors and loaded by the engine, 4 univariate series of 512
    steps, horizon 64: quantiles within 1e-3; the device encoder's output after each layer (fed the
    same tokens) within 1e-4."""
    import torch

    import tests.golden.make_config0 as mk
    from jitcast_amd import chronos2_model as cm
    from jitcast_amd import synthetic

    g = np.load(mk.OUT)
    w = synthetic.c2_portable_weights(mk.CONFIG0, seed=0)
    ck.write_chronos2(tmp_path, mk.CONFIG0, w)
    with HipChronos2Engine.load(tmp_path) as eng:
        got = eng.forecast([TimeSeries.univariate(row) for row in g["inputs"]], mk.HORIZON)
        q = np.stack([f.values[0] for f in got])
        err = oracle.rel_max_error(q, g["quantiles"])
        print(f"config 0 quantiles rel err {err:.2e}", flush=True)
        assert err <= 1e-3
        c = mk.CONFIG0
        lay = cm.layout(c, g["inputs"], np.arange(4), None, h=mk.HORIZON // c.patch_size)
        tok, _, _ = oracle.c2_prep(lay.window, lay.future, lay.nc, lay.h, c.patch_size, c.time_encoding_scale,
                                   c.use_arcsinh)
        gs, ge = cm.chronos2.group_bounds(lay.group)
        model = eng.forward_pass().model
        dev = model.dev
        seen = {}
        model.forward_raw(torch.from_numpy(tok).to(dev), torch.from_numpy(lay.live.reshape(-1)).to(dev),
                          torch.from_numpy(gs).to(dev), torch.from_numpy(ge).to(dev), lay.rows, lay.nc, lay.h,
                          sink=lambda name, x: seen.setdefault(name, x.cpu().numpy()))
        errs = [oracle.rel_max_error(seen[f"layer{i}"], g["layers"][i]) for i in range(c.num_layers)]
        print("config 0 layers rel err " + " ".join(f"{e:.1e}" for e in errs), flush=True)
        assert max(errs) <= 1e-4


@pytest.mark.parametrize("cross,max_tokens", [(True, 131072), (False, 500)])
def test_engine_cross_learning_and_token_splits(gpu, oracle, checkpoint, cross, max_tokens):
    """Through the engine, against the restatement over the oracle's forward: cross-learning (one
    group per batch, so the group attention runs over every row of the batch), and a token budget
    that splits each pass into several by whole groups. fp32: every call within 1e-4, forecasts
    within 1e-3."""
    from jitcast_amd.pipeline import Options

    print(f"case engine cross={cross} max_tokens={max_tokens}", flush=True)
    horizon = 40
    series = _mixed_batch(17, 30, horizon)
    _, w = ck.load_chronos2(checkpoint)
    calls = []
    with HipChronos2Engine.load(checkpoint, dtype="f32") as eng:
        fwd = eng.forward_pass()
        ofwd = _oracle_forward(oracle, C, w)

        def checked(inp):
            out = fwd(inp)
            err = oracle.rel_max_error(out, ofwd(inp.context, inp.group, inp.future_covariates, inp.output_patches))
            calls.append((inp.rows(), len(np.unique(inp.group)), err))
            print(f"  call{len(calls) - 1} rows={inp.rows()} groups={calls[-1][1]} rel err {err:.2e}", flush=True)
            return out

        pipe = eng.pipeline().with_options(Options.defaults(C).with_cross_learning(cross)).with_max_tokens(max_tokens)
        pipe.forward = checked
        got = pipe.forecast([TimeSeries(t, p, k) for t, p, k in series], horizon)
    exp = ref.forecast(C, _oracle_forward(oracle, C, w), series, horizon, cross_learning=cross, max_tokens=max_tokens)
    assert calls and max(e for _, _, e in calls) <= 1e-4
    if cross:
        assert all(g == 1 for _, g, _ in calls), "one group per batch"
    else:
        assert len(calls) > 1, "the budget splits the pass"
    err = max(oracle.rel_max_error(g.values, e) for g, e in zip(got, exp))
    print(f"  forecasts rel err {err:.2e} (bar 1e-3)", flush=True)
    assert err <= 1e-3
