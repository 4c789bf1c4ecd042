"""The Timestral block's shape bucketing and plan cache on the GPU (TimestralForward.java:81-99,
135-252): a block padded to its bucket (leading empty patches, empty series of their own) forecasts
its real rows as the unpadded block does, and forecasts replayed from captured plans (one hipGraph
per Shape(rows, encoder, horizon, covariates)) equal the eager forward bit for bit across shapes,
with eager work between replays and an eviction."""
import numpy as np
import pytest
import torch

from jitcast_amd import timestral_model as tm

pytestmark = pytest.mark.gpu

C = tm.TimestralConfig(patch_size=8, d_model=64, num_heads=2, mlp_hidden_dim=96, layers=((True, False), (True, False)),
                       quantiles=(0.1, 0.5, 0.9), block_size=4)


def _block(seed, rows, patches, h, covariates):
    r = np.random.default_rng(seed)
    t = patches * C.patch_size
    x = (20 + 4 * np.sin(np.arange(t) / 5.0)[None, :] + r.standard_normal((rows, t))).astype(np.float32)
    obs = r.random((rows, t)) > 0.1
    obs[0, : t // 3] = False
    per = 3
    group = (np.arange(rows) // per).astype(np.int32)
    role = fut = fut_mask = None
    if covariates:
        role = np.array([i % per for i in range(rows)], np.int32)
        fut = r.standard_normal((rows, h * C.patch_size)).astype(np.float32)
        fut_mask = np.zeros((rows, h * C.patch_size), bool)
        fut_mask[role == 2] = True
    return x, obs, group, h, role, fut, fut_mask


_W = tm.random_weights(C, seed=11, std=0.1)


@pytest.mark.parametrize("covariates", [False, True])
def test_bucketed_block_forecasts_its_rows_unchanged(gpu, covariates):
    print(f"case ts bucketing covariates={covariates}", flush=True)
    blk = _block(3, 11, 37, 2, covariates)  # pads to 12 rows and 40 patches
    a = tm.HipTimestralModel(C, _W, buckets=True).predict_block(*blk)
    b = tm.HipTimestralModel(C, _W, buckets=False).predict_block(*blk)
    assert a.shape == b.shape == (11, 2 * C.patch_size, 3)
    d = float(np.max(np.abs(a.astype(np.float64) - b)) / np.max(np.abs(b)))
    print(f"  bucketed vs exact: max rel diff {d:.2e}, bit-identical: {np.array_equal(a, b)}", flush=True)
    # The leading empty patches shift the real keys inside the time attention's 64-key blocks, which
    # reorders its fp32 sums: about 1e-6 of the forecasts (measured 1.3e-6 and 1.8e-6 here).
    assert d <= 1e-5
    # padded rows alone (the patch count already a bucket) change nothing: every kernel computes a
    # series' rows the same way wherever they sit
    blk = _block(4, 11, 40, 2, covariates)  # 40 patches is a bucket; 11 rows pad to 12
    a = tm.HipTimestralModel(C, _W, buckets=True).predict_block(*blk)
    b = tm.HipTimestralModel(C, _W, buckets=False).predict_block(*blk)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_planned_blocks_match_eager(gpu, dt):
    print(f"case ts plans {dt}", flush=True)
    eager = tm.HipTimestralModel(C, _W, dtype=dt, buckets=False, max_plans=0)
    planned = tm.HipTimestralModel(C, _W, dtype=dt, buckets=False, max_plans=2)
    try:
        runs = [(6, 12, 2, False), (9, 7, 1, True), (6, 12, 2, False), (3, 16, 3, False), (6, 12, 2, False)]
        for k, (rows, patches, h, cov) in enumerate(runs):
            blk = _block(20 + k, rows, patches, h, cov)
            got = planned.predict_block(*blk)
            exp = eager.predict_block(*blk)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(got, exp)
        # shapes A = (6, 12, 2), B = (9, 7 + 1, 1, cov), C = (3, 16, 3): A, B, A (hit), C evicts B, A (hit)
        assert [k[:3] for k in planned.plans.keys()] == [(3, 16, 3), (6, 12, 2)]
    finally:
        planned.close()
    assert planned.plans.keys() == []
    assert eager.plans is None


def test_plans_on_by_default(gpu):
    """The reference's default: eight plans per model (timestral.tornado.plans, docs/CONFIGURATION.md:131),
    here -Dtimestral.hip.plans; 0 runs eagerly."""
    from jitcast_amd import options

    m = tm.HipTimestralModel(C, _W)
    assert m.plans is not None and m.plans.max_plans == 8
    options.set_property("timestral.hip.plans", "0")
    try:
        assert tm.HipTimestralModel(C, _W).plans is None
    finally:
        options.set_property("timestral.hip.plans", None)
