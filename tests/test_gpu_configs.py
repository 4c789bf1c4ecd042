"""GPU parity at the benchmark configurations' model shapes, against the oracle.

Config 3: the Timestral 123M-class attention stack (d_model 768, 12 x 64 heads, 12 layers of
RMSNorm -> q|k|v -> RoPE (half the head) -> time attention -> sigmoid gate -> output projection
added to x), N(0, 0.02) weights, x ~ N(0, 1) embeddings, bidirectional attention over valid keys
(every row a known covariate: BlockLayout.timeAllowed, J/timestral/BlockLayout.java:209-221) with
per-series left padding masked. The bf16 and fp16 variants (storage-type GEMM operands and time
attention, fp32 accumulation and residual stream) are held to 2e-2 against the fp32 oracle, fp32 to
1e-4. Two series of config 3's 1,024 tokens run against the oracle; the full 64-series batch is
checked through properties the path must keep (finite outputs, equivariance under permuting the
series).

Config 4: the Chronos-2 120M-class forecast (d_model 768, 12 x 64, 12 layers, d_ff 3072, patch 16,
21 quantiles), groups of 4 target series and 1 known-future covariate of 2,048 steps, horizon 64.
Two groups run against the oracle's CpuChronos2.forward restatement (fp32 encoder and the f16x3
encoder, fp16 GEMMs over three-term splits of every fp32 operand: quantiles within 1e-3; the bf16 and
fp16 encoders' errors are reported and held to 2e-2); the full 1,024-group request is checked for
finite quantiles and equivariance under permuting the groups (in blocks of 16: whole 16-row tiles).
"""
import numpy as np
import pytest
import torch

from jitcast_amd import chronos2_model as cm
from jitcast_amd import rng, synthetic
from jitcast_amd import timestral_model as tm

pytestmark = pytest.mark.gpu

# config 3's attention stack: one time-attention sublayer per layer, gates on, the MLP left out
C3 = tm.TimestralConfig(layers=((True,),) * 12)
C3_TOL = {"f32": 1e-4, "bf16": 2e-2, "fp16": 2e-2}
# The stack moves x by under 2% of max|x| at these weights, so the output bar alone would pass a
# broken attention: the update the 12 layers add (x_out - x_in) is held to its own bar too.
C3_UPDATE_TOL = {"f32": 1e-4, "bf16": 5e-2, "fp16": 2e-2}
_cache = {}


def _c3_case(rows: int, n: int = 1024, seed: int = 0):
    """x ~ N(0, 1) [rows*n, 768], left padding U{0..256} tokens per series (keys before the first
    observed patch invalid), positions counted from the first observed patch."""
    x = rng.normal(rng.stream_seed(seed, 30), rows * n * C3.d_model).reshape(rows * n, C3.d_model)
    starts = rng.randint(rng.stream_seed(seed, 31), rows, 0, 256)
    t = np.arange(n)[None, :]
    kv = (t >= starts[:, None]).astype(np.int32)
    position = (t - starts[:, None]).astype(np.int32)
    known = np.ones(rows, np.int32)
    return x, kv, known, position


def _c3_weights():
    if "c3w" not in _cache:
        _cache["c3w"] = tm.random_weights(C3, seed=0, std=0.02)
    return _cache["c3w"]


def _c3_device(model, x, kv, known, position, rows, n):
    dev = model.dev
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    xd = up(x)
    model.encoder(xd, up(kv.reshape(-1)), up(known), up((position + n).reshape(-1)), None, None, None, False, rows, n,
                  0, mlp=False)
    return xd


@pytest.mark.parametrize("dt", ["f32", "bf16", "fp16"])
def test_config3_attention_stack_matches_oracle(gpu, oracle, dt):
    rows, n = 2, 1024
    print(f"case config 3 stack {dt}: {rows} series x {n} tokens, 12 layers, d768, 12x64", flush=True)
    x, kv, known, position = _c3_case(rows, n)
    w = _c3_weights()
    if "c3exp" not in _cache:
        _cache["c3exp"] = oracle.ts_encoder(x, w, kv, known, position, np.arange(rows, dtype=np.int32),
                                            np.zeros(rows, np.int32), 0, rows, n, n, 0, C3.num_heads, C3.head_dim,
                                            C3.rope_dim, C3.norm_eps, C3.rope_theta, mlp=False)
    exp = _cache["c3exp"]
    model = tm.HipTimestralModel(C3, w, dtype=dt)
    got = _c3_device(model, x, kv, known, position, rows, n)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    err = oracle.rel_max_error(got, exp)
    upd = oracle.rel_max_error(got - x, exp - x)
    drift = oracle.rel_max_error(exp, x)
    print(f"  rel err {err:.3e} (bar {C3_TOL[dt]:.0e}); update rel err {upd:.3e} (bar {C3_UPDATE_TOL[dt]:.0e}); "
          f"the stack moves x by {drift:.3e}", flush=True)
    assert err <= C3_TOL[dt]
    assert upd <= C3_UPDATE_TOL[dt]


def test_config3_full_batch_properties(gpu):
    """All 64 series of config 3 in bf16: finite, and permuting the series permutes the output bit for
    bit (each series' attention, norms and GEMM rows are computed independently of its slot)."""
    rows, n = 64, 1024
    print(f"case config 3 stack bf16 full batch: {rows} x {n}", flush=True)
    x, kv, known, position = _c3_case(rows, n, seed=1)
    model = tm.HipTimestralModel(C3, _c3_weights(), dtype="bf16")
    a = _c3_device(model, x, kv, known, position, rows, n).cpu().numpy()
    perm = np.random.default_rng(2).permutation(rows)
    tok = lambda v: v.reshape(rows, n, -1)[perm].reshape(rows * n, -1)  # noqa: E731
    b = _c3_device(model, tok(x), kv[perm], known[perm], position[perm], rows, n).cpu().numpy()
    assert np.isfinite(a).all()
    np.testing.assert_array_equal(tok(a), b)


def _c3_block_config():
    # the full block (time + variate attention, SwiGLU MLP, head) at config 3's model dims
    return tm.TimestralConfig()


def test_config3_block_forward_bf16_matches_oracle(gpu, oracle):
    """The whole Timestral block forward (embedding, 12 layers of time + variate attention with gates
    and the SwiGLU MLP, head) at config 3's model dims in the FP16-GEMM mode (bf16), against the fp32
    oracle within 2e-2, and in fp32 within 1e-4; 2 series of 255 context patches + 1 forecast patch."""
    from jitcast_amd import chronos2, timestral

    c = _c3_block_config()
    rows, enc, h = 2, 255, 1
    print(f"case config 3 block forward: {rows} series x {enc}+{h} tokens, d768, 12 layers", flush=True)
    w = tm.random_weights(c, seed=4, std=0.02)
    r = np.random.default_rng(5)
    tok = r.standard_normal((rows * enc, 2 * c.patch_size)).astype(np.float32)
    obs = np.ones((rows, enc * c.patch_size), bool)
    obs[0, : 40 * c.patch_size] = False
    group = np.arange(rows, dtype=np.int32)
    enc_l, _, kv, known, pos = timestral.block_layout(obs, group, h, c.patch_size)
    assert enc_l == enc
    exp = oracle.ts_forward_raw(tok, w, kv, known, pos - enc, group, np.zeros(rows, np.int32), 0, rows, enc, enc, h,
                                c.num_heads, c.head_dim, c.rope_dim, c.norm_eps, c.rope_theta)
    gs, ge = chronos2.group_bounds(group)
    for dt, bar in (("f32", 1e-4), ("bf16", 2e-2)):
        model = tm.HipTimestralModel(c, w, dtype=dt)
        up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(model.dev)  # noqa: E731
        raw = model.forward_raw(up(tok), up(kv.reshape(-1)), up(known), up(pos.reshape(-1)), up(gs), up(ge), None, False,
                                rows, enc, h)
        torch.cuda.synchronize()
        err = oracle.rel_max_error(raw.cpu().numpy(), exp)
        print(f"  {dt} raw rel err {err:.3e} (bar {bar:.0e})", flush=True)
        assert err <= bar
        del model


C4 = cm.Chronos2Config()  # 120M-class: d_model 768, 12 x 64, 12 layers, d_ff 3072, 21 quantiles


def _c4_weights():
    if "c4w" not in _cache:
        _cache["c4w"] = cm.random_weights(C4, seed=0)
    return _cache["c4w"]


@pytest.mark.parametrize("dt", ["f32", "f16x3", "bf16", "fp16"])
def test_config4_forecast_matches_oracle(gpu, oracle, dt):
    groups, h = 2, 4
    print(f"case config 4 forecast {dt}: {groups} groups x 5 rows x 2048 steps, h={h}, 120M-class", flush=True)
    ctx, group, fut, _ = synthetic.c2_forecast_config4(groups=groups, seed=7)
    w = _c4_weights()
    if "c4exp" not in _cache:
        # the oracle's own ModelLayout.of, ModelPrep and forward (oracle.c2_model_forward), not the product's
        _cache["c4exp"] = oracle.c2_model_forward(C4, w, ctx, group, fut, h)
    exp = _cache["c4exp"]
    model = cm.HipChronos2Model(C4, w, dtype=dt)
    got = model.forecast(ctx, group, fut, h=h)
    err = oracle.rel_max_error(got, exp)
    bar = 1e-3 if dt in ("f32", "f16x3") else 2e-2
    print(f"  quantiles rel err {err:.3e} (bar {bar:.0e})", flush=True)
    assert got.shape == (groups * 5, C4.num_quantiles, h * C4.patch_size)
    assert err <= bar


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_config4_call_reproducible(gpu, dt):
    """One of config 4's forward calls (52 groups x 5 rows x 2048 steps: 260 rows of 133 tokens through
    the 120M-class encoder) forecast eagerly and from its plan, three times each, with another engine's
    GEMMs (other hipBLASLt algorithms) run in between: every forecast is bit-identical to the first. A
    plan replays the eager task graph (J/chronos2/tornado/Chronos2Forward.java:292-300)."""
    print(f"case config 4 call reproducible {dt}: 52 groups x 5 rows, h=4", flush=True)
    ctx, group, fut, _ = synthetic.c2_forecast_config4(groups=52, seed=11)
    w = _c4_weights()
    eager = cm.HipChronos2Model(C4, w, dtype=dt)
    planned = cm.HipChronos2Model(C4, w, dtype=dt, max_plans=1)
    other = cm.HipChronos2Model(C4, w, dtype="f16x3" if dt == "bf16" else "bf16")
    try:
        first = eager.forecast(ctx, group, fut, h=4)
        assert np.isfinite(first).all()
        for k in range(3):
            other.forecast(ctx[:25], group[:25], fut[:25], h=4)
            p = planned.forecast(ctx, group, fut, h=4)
            e = eager.forecast(ctx, group, fut, h=4)
            torch.cuda.synchronize()
            print(f"  round {k}: plan differs in {int((p != first).sum())} values, eager in {int((e != first).sum())}",
                  flush=True)
            np.testing.assert_array_equal(p, first)
            np.testing.assert_array_equal(e, first)
    finally:
        planned.close()


def test_config4_full_request_properties(gpu):
    """Config 4's full request (1,024 groups, 5,120 rows) through the fp32 encoder: finite quantiles,
    and permuting the groups in blocks of 16 permutes the forecasts bit for bit. The GEMMs and the
    time attention compute a row independently of its slot (no GEMM tile's k range is split over
    workgroups). Group attention packs the small groups that start in a 16-row tile into one job,
    so a group's sums depend on its place in its tile; 16 groups of 5 are 80 rows, five whole
    tiles, so moving blocks of them keeps every group's place while every row changes GEMM tiles."""
    print("case config 4 full request fp32: 1024 groups x 5 rows x 2048 steps", flush=True)
    ctx, group, fut, _ = synthetic.c2_forecast_config4()
    model = cm.HipChronos2Model(C4, _c4_weights(), dtype="f32")
    a = model.forecast(ctx, group, fut, h=4)
    assert np.isfinite(a).all()
    bperm = np.random.default_rng(3).permutation(1024 // 16)
    gperm = (bperm[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    rows = (gperm[:, None] * 5 + np.arange(5)[None, :]).reshape(-1)
    b = model.forecast(ctx[rows], group[rows], fut[rows], h=4)
    d = float(np.max(np.abs(a[rows].astype(np.float64) - b)) / np.max(np.abs(b)))
    print(f"  permuted groups: max rel diff {d:.2e}", flush=True)
    np.testing.assert_array_equal(a[rows], b)
