"""GPU parity of the Timestral block's device pieces (jc_ts_residual, jc_ts_assemble,
jc_ts_gather_decoder, jc_swiglu) and of the whole device forward (HipTimestralModel.forward_raw:
TimestralForward.Plan's task order, J/timestral/tornado/TimestralForward.java:327-382) against the
oracle's CpuTimestral restatement (pinned in test_oracle_ts_forward.py). Bars: fp32 within 1e-4 by
the reference's metric (the raw head outputs, before the quantile map); moves bit-exact; the
storage-type SwiGLU within one rounding to the type."""
import numpy as np
import pytest
import torch

from jitcast_amd import JitcastArgumentError, _lib, chronos2, timestral
from jitcast_amd import timestral_model as tm
from tests import cases

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dt)


def _i32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


# f = 96: the 16-byte path for every type; 36: 16-byte for fp32, per element for bf16 / fp16; 35: per
# element for every type
@pytest.mark.parametrize("f", [96, 36])
def test_swiglu_x3_is_the_split_of_the_fp32_swiglu(gpu, f):
    """jc_swiglu with JC_F16X3 (fp32 up, fp16 act [tokens, 3f]) writes the A-operand split [hi | hi |
    lo] of the fp32 SwiGLU: both hi copies equal, and hi + lo within 2^-21 of the fp32 jc_swiglu's
    result plus fp16's subnormal spacing (the split's 2^-22 and an ulp of fp32 SwiGLU's own rounding,
    which the two kernels may compile differently). f not a multiple of 4 is rejected."""
    r = np.random.default_rng(8)
    tokens = 301
    ut = _t((3 * r.standard_normal((tokens, 2 * f))).astype(np.float32), torch.float32)
    act = torch.empty(tokens, f, dtype=torch.float32, device=DEV)
    act3 = torch.empty(tokens, 3 * f, dtype=torch.float16, device=DEV)
    ctx = chronos2.context(0)
    _lib.call("jc_swiglu", ctx.handle, chronos2._ptr(ut), chronos2._ptr(act), tokens, f, _lib.JC_F32)
    _lib.call("jc_swiglu", ctx.handle, chronos2._ptr(ut), chronos2._ptr(act3), tokens, f, _lib.JC_F16X3)
    torch.cuda.synchronize()
    got = act3.cpu().numpy()
    ref = act.cpu().numpy().astype(np.float64)
    np.testing.assert_array_equal(got[:, :f].view(np.uint16), got[:, f:2 * f].view(np.uint16))
    recon = got[:, :f].astype(np.float64) + got[:, 2 * f:].astype(np.float64)
    err = np.abs(recon - ref)
    print(f"  swiglu x3: max |hi + lo - fp32| / |fp32| {np.max(err / np.maximum(np.abs(ref), 1e-30)):.2e}", flush=True)
    assert np.all(err <= 2 ** -21 * np.abs(ref) + 2 ** -24)
    with pytest.raises(JitcastArgumentError):
        _lib.call("jc_swiglu", ctx.handle, chronos2._ptr(ut), chronos2._ptr(act3), tokens, 35, _lib.JC_F16X3)


@pytest.mark.parametrize("f", [96, 36, 35])
@pytest.mark.parametrize("dt", ["f32", "bf16", "fp16"])
def test_swiglu_matches_oracle(gpu, oracle, dt, f):
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}[dt]
    code = {"f32": _lib.JC_F32, "bf16": _lib.JC_BF16, "fp16": _lib.JC_F16}[dt]
    r = np.random.default_rng(7)
    tokens = 301
    up = (3 * r.standard_normal((tokens, 2 * f))).astype(np.float32)
    up[0, 0], up[0, f] = 1e5, 1e5  # saturates in fp16
    ut = _t(up, tdt)
    act = torch.empty(tokens, f, dtype=tdt, device=DEV)
    ctx = chronos2.context(0)
    _lib.call("jc_swiglu", ctx.handle, chronos2._ptr(ut), chronos2._ptr(act), tokens, f, code)
    torch.cuda.synchronize()
    exp = oracle.swiglu(ut.float().cpu().numpy(), f)
    got = act.float().cpu().numpy()
    if dt == "f32":
        assert oracle.rel_max_error(got, exp) <= 1e-6
    else:
        lim = 65504.0 if dt == "fp16" else 3.0e38
        exp_c = np.clip(exp, -lim, lim)
        assert np.all(np.abs(got - exp_c) <= np.abs(exp_c) * 2.0 ** -7 + 1e-30)
        if dt == "fp16":
            assert got[0, 0] == np.float32(65504.0)


def test_assemble_and_gather(gpu):
    r = np.random.default_rng(8)
    rows, enc, h, d = 5, 7, 3, 24
    n = enc + h
    emb = r.standard_normal((rows * enc, d)).astype(np.float32)
    query = r.standard_normal(d).astype(np.float32)
    x = torch.empty(rows * n, d, device=DEV)
    ctx = chronos2.context(0)
    p = chronos2._ptr
    et, qt = _t(emb), _t(query)
    _lib.call("jc_ts_assemble", ctx.handle, p(et), p(qt), p(x), rows, enc, n, d)
    dec = torch.empty(rows * h, d, device=DEV)
    _lib.call("jc_ts_gather_decoder", ctx.handle, p(x), p(dec), rows, enc, n, h, d)
    torch.cuda.synchronize()
    exp = np.empty((rows, n, d), np.float32)
    exp[:, :enc] = emb.reshape(rows, enc, d)
    exp[:, enc:] = query
    np.testing.assert_array_equal(x.cpu().numpy(), exp.reshape(rows * n, d))
    np.testing.assert_array_equal(dec.cpu().numpy(), exp[:, enc:].reshape(rows * h, d))
    with pytest.raises(_lib.JitcastArgumentError):
        _lib.call("jc_ts_gather_decoder", ctx.handle, p(x), p(dec), rows, enc, n, h + 1, d)


def test_residual_matches_oracle(gpu, oracle):
    c = tm.TimestralConfig(patch_size=8, d_model=32, num_heads=2, mlp_hidden_dim=48, layers=((True,),),
                           quantiles=(0.1, 0.5, 0.9))
    w = tm.random_weights(c, seed=4, std=0.3)
    r = np.random.default_rng(9)
    m = 37
    x = r.standard_normal((m, 2 * c.patch_size)).astype(np.float32)
    out = torch.empty(m, c.d_model, device=DEV)
    scratch = torch.empty(m, 4 * c.d_model, device=DEV)
    wt = {k: _t(v) for k, v in w.items() if k.startswith("embed")}
    p = chronos2._ptr
    ctx = chronos2.context(0)
    xt = _t(x)
    _lib.call("jc_ts_residual", ctx.handle, p(xt), m, 2 * c.patch_size, p(wt["embed_hidden_w"]), p(wt["embed_hidden_b"]),
              p(wt["embed_output_w"]), p(wt["embed_output_b"]), p(wt["embed_residual_w"]), p(wt["embed_residual_b"]),
              4 * c.d_model, c.d_model, p(scratch), p(out))
    torch.cuda.synchronize()
    exp = oracle.ts_residual(x, w, "embed")
    assert oracle.rel_max_error(out.cpu().numpy(), exp) <= 1e-5


CASES = [
    # name, config, rows, groups, enc, h, covariates
    ("tiny", tm.TimestralConfig(patch_size=8, d_model=32, num_heads=2, mlp_hidden_dim=48,
                                layers=((True, False), (False, True)), quantiles=(0.1, 0.5, 0.9)), 6, 2, 5, 2, True),
    ("tiny-univariate", tm.TimestralConfig(patch_size=8, d_model=32, num_heads=2, mlp_hidden_dim=48,
                                           layers=((True,), (True,)), quantiles=(0.1, 0.5, 0.9), time_attn_gate=False),
     4, 4, 9, 3, False),
    ("d128", tm.TimestralConfig(patch_size=16, d_model=128, num_heads=2, mlp_hidden_dim=256,
                                layers=((True, False), (True, False)), quantiles=(0.1, 0.2, 0.5, 0.8, 0.9)),
     12, 3, 40, 4, True),
]


@pytest.mark.parametrize("name,c,rows,groups,enc,h,covariates", CASES, ids=[x[0] for x in CASES])
def test_forward_matches_oracle(gpu, oracle, name, c, rows, groups, enc, h, covariates):
    print(f"case ts forward {name} rows={rows} enc={enc} h={h} covariates={covariates}", flush=True)
    ll = enc - h if covariates else enc
    kv, known, position = cases.ts_layout(17, rows, enc, ll, h, known_frac=0.3 if covariates else 0.0)
    per = rows // groups
    group = np.repeat(np.arange(groups), per).astype(np.int32)
    role = np.tile(np.array([0] + [1 + (i % 2) for i in range(per - 1)], np.int32), groups) if covariates \
        else np.zeros(rows, np.int32)
    w = tm.random_weights(c, seed=5, std=0.1)
    r = np.random.default_rng(6)
    tok = r.standard_normal((rows * enc, 2 * c.patch_size)).astype(np.float32)
    model = tm.HipTimestralModel(c, w)
    gs, ge = chronos2.group_bounds(group)
    raw = model.forward_raw(_t(tok), _i32(kv.reshape(-1)), _i32(known), _i32((position + enc).reshape(-1)), _i32(gs),
                            _i32(ge), _i32(role) if covariates else None, covariates, rows, enc, h)
    torch.cuda.synchronize()
    exp = oracle.ts_forward_raw(tok, w, kv, known, position, group, role, covariates, rows, enc, ll, h, c.num_heads,
                                c.head_dim, c.rope_dim, c.norm_eps, c.rope_theta)
    err = oracle.rel_max_error(raw.cpu().numpy(), exp)
    print(f"  raw rel err {err:.3e}", flush=True)
    assert err <= 1e-4


def _oracle_block(oracle, c, x, obs, group, h, role, fut, fut_mask):
    """CpuTimestral.predictBlock end to end on the oracle's pieces (its BlockLayout, BlockPrep,
    forward and finish): nothing of the product's host code."""
    ps = c.patch_size
    window, wobs, enc, cov, kv, known, position, ll = oracle.ts_block_layout(
        x, obs, group, h, ps, role, fut, fut_mask, c.covariate_enabled, c.attend_missing, c.block_size)
    tok, _, loc, scale = oracle.ts_block_prep(window, wobs, known, ps, c.minimum_scale, c.use_asinh)
    rows = x.shape[0]
    raw = oracle.ts_forward_raw(tok, tm_weights(c), kv, known, position, group,
                                np.asarray(role, np.int32) if cov else np.zeros(rows, np.int32), cov, rows, enc, ll, h,
                                c.num_heads, c.head_dim, c.rope_dim, c.norm_eps, c.rope_theta)
    return oracle.ts_block_finish(raw, loc, scale, ll, h, ps, c.quantiles, c.median_index, c.quantile_width_factor,
                                  c.use_asinh)


_W = {}


def tm_weights(c):
    if c not in _W:
        _W[c] = tm.random_weights(c, seed=11, std=0.1)
    return _W[c]


@pytest.mark.parametrize("covariates", [False, True])
def test_predict_block_matches_oracle(gpu, oracle, covariates):
    """BlockLayout + BlockPrep + device forward + finish against the oracle's CpuTimestral restatement,
    quantiles within 1e-3 (the north star's end-to-end bar)."""
    c = tm.TimestralConfig(patch_size=8, d_model=64, num_heads=2, mlp_hidden_dim=96,
                           layers=((True, False), (True, False)), quantiles=(0.1, 0.5, 0.9), block_size=4)
    print(f"case predict_block covariates={covariates}", flush=True)
    r = np.random.default_rng(12)
    rows, t, h = 6, 48, 3
    x = (20 + 4 * np.sin(np.arange(t) / 5.0)[None, :] + r.standard_normal((rows, t))).astype(np.float32)
    obs = r.random((rows, t)) > 0.1
    obs[1, :20] = False
    group = np.array([0, 0, 0, 1, 1, 1], np.int32)
    role = np.array([0, 1, 2, 0, 2, 1], np.int32) if covariates else None
    fut = fut_mask = None
    if covariates:
        fut = r.standard_normal((rows, h * 8)).astype(np.float32)
        fut_mask = np.zeros((rows, h * 8), bool)
        fut_mask[role == 2] = True
    model = tm.HipTimestralModel(c, tm_weights(c))
    got = model.predict_block(x, obs, group, h, role, fut, fut_mask)
    exp = _oracle_block(oracle, c, x, obs, group, h, role, fut, fut_mask)
    assert got.shape == (rows, h * 8, 3)
    err = oracle.rel_max_error(got, exp)
    print(f"  quantiles rel err {err:.3e}", flush=True)
    assert err <= 1e-3
    assert np.all(np.diff(got, axis=2) >= 0)  # non-crossing


@pytest.mark.parametrize("dt,bar", [("bf16", 2e-2), ("fp16", 2e-2), ("f16x3", 1e-4)])
@pytest.mark.parametrize("name,c,rows,groups,enc,h,covariates", [CASES[0], CASES[2]], ids=["tiny", "d128"])
def test_forward_lowp_matches_fp32_oracle(gpu, oracle, dt, bar, name, c, rows, groups, enc, h, covariates):
    """The FP16-GEMM mode (storage-type GEMM operands and time attention, fp32 accumulation and
    residual stream) against the fp32 oracle on the same unrounded weights: within 2e-2. f16x3 (fp32
    activations, every GEMM over three-term fp16 splits): within fp32's bar, 1e-4."""
    print(f"case ts forward {dt} {name}", flush=True)
    ll = enc - h if covariates else enc
    kv, known, position = cases.ts_layout(17, rows, enc, ll, h, known_frac=0.3 if covariates else 0.0)
    per = rows // groups
    group = np.repeat(np.arange(groups), per).astype(np.int32)
    role = np.tile(np.array([0] + [1 + (i % 2) for i in range(per - 1)], np.int32), groups) if covariates \
        else np.zeros(rows, np.int32)
    w = tm.random_weights(c, seed=5, std=0.1)
    r = np.random.default_rng(6)
    tok = r.standard_normal((rows * enc, 2 * c.patch_size)).astype(np.float32)
    model = tm.HipTimestralModel(c, w, dtype=dt)
    gs, ge = chronos2.group_bounds(group)
    raw = model.forward_raw(_t(tok), _i32(kv.reshape(-1)), _i32(known), _i32((position + enc).reshape(-1)), _i32(gs),
                            _i32(ge), _i32(role) if covariates else None, covariates, rows, enc, h)
    torch.cuda.synchronize()
    exp = oracle.ts_forward_raw(tok, w, kv, known, position, group, role, covariates, rows, enc, ll, h, c.num_heads,
                                c.head_dim, c.rope_dim, c.norm_eps, c.rope_theta)
    err = oracle.rel_max_error(raw.cpu().numpy(), exp)
    print(f"  raw rel err {err:.3e}", flush=True)
    assert err <= bar
