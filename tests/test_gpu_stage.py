"""GPU parity of the Chronos-2 encoder layer around the attention cores (through the C ABI):
jc_linear (Kernels.gemm's flags), jc_rms_norm (Kernels.rmsNorm) and jc_c2_layer (the per-layer stage
of Chronos2Forward.Plan, Chronos2Forward.java:258-286) against the oracle.

Bar: max relative error (the reference's metric) <= 1e-4 for the fp32 layer; the GEMM and the norm
alone are held to 1e-5. The GEMM and layer tests run on both GEMM paths: hipBLASLt (the default) and
the library's own MFMA kernels.
"""
import numpy as np
import pytest
import torch

from jitcast_amd import JitcastArgumentError, _lib, chronos2
from tests import cases
from tests.test_oracle_ops import _layer_weights

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 1e-4


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _epilogue(y, c0, bias, flags):
    y = y.astype(np.float64)
    if bias is not None:
        y = y + bias.astype(np.float64)
    if flags & chronos2.GEMM_SILU:
        y = y / (1 + np.exp(-y))
    if flags & chronos2.GEMM_RELU:
        y = np.maximum(y, 0)
    if flags & chronos2.GEMM_ACCUMULATE:
        y = y + c0
    return y


@pytest.mark.parametrize("m,n,k", [(1, 16, 16), (37, 100, 64), (129, 130, 784), (300, 257, 48), (256, 128, 128)])
@pytest.mark.parametrize("flags,bias", [(0, False), (0, True), (chronos2.GEMM_RELU, True),
                                        (chronos2.GEMM_ACCUMULATE, False), (chronos2.GEMM_ACCUMULATE, True),
                                        (chronos2.GEMM_SILU, True), (chronos2.GEMM_RELU | chronos2.GEMM_ACCUMULATE, False)])
def test_linear_matches_oracle(gpu, oracle, gemm_path, m, n, k, flags, bias):
    print(f"case m={m} n={n} k={k} flags={flags} bias={bias}", flush=True)
    r = np.random.default_rng(m * 7 + n * 3 + k + flags)
    a = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = r.standard_normal(n).astype(np.float32) if bias else None
    c0 = r.standard_normal((m, n)).astype(np.float32)
    c = _t(c0)
    chronos2.linear(_t(a), _t(w), c, bias=_t(b) if bias else None, flags=flags)
    torch.cuda.synchronize()
    exp = _epilogue(oracle.linear(a, w), c0, b, flags)
    assert oracle.rel_max_error(c.cpu().numpy(), exp) <= 1e-5


@pytest.mark.parametrize("dt,n,k,flags,out", [
    ("f32", 2304, 768, 0, "f32"), ("f32", 768, 3072, chronos2.GEMM_ACCUMULATE, "f32"),
    ("bf16", 2304, 768, 0, "lp"), ("bf16", 3072, 768, chronos2.GEMM_RELU, "lp"),
    ("bf16", 768, 768, chronos2.GEMM_ACCUMULATE, "f32")])
def test_gemm_rows_are_independent(gpu, gemm_path, dt, n, k, flags, out):
    """Config 4's GEMM shapes (m = 260 rows x 133 tokens = 34,580): permuting the rows of A (and of C
    for ACCUMULATE) permutes the rows of C bit for bit, and a repeated call gives the same bits. Each
    tile of C is then one workgroup's fixed-order sum over k, wherever a row sits: the property that
    keeps forecasts reproducible. A GEMM that splits a tile's k range over workgroups and adds the
    partial tiles (hipBLASLt's Stream-K kernels given a workspace) changes a row's rounding with its
    position."""
    m = 260 * 133
    print(f"case {dt} m={m} n={n} k={k} flags={flags} out={out}", flush=True)
    r = np.random.default_rng(n + k + flags)
    tdt = torch.float32 if dt == "f32" else LP[dt]
    a = _t(r.standard_normal((m, k)).astype(np.float32)).to(tdt)
    w = _t((r.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)).to(tdt)
    c0 = _t(r.standard_normal((m, n)).astype(np.float32))
    perm = torch.from_numpy(np.random.default_rng(7).permutation(m)).to(DEV)
    run = chronos2.linear if dt == "f32" else chronos2.linear_lp

    def gemm(a_, c_init):
        c = c_init.clone() if out == "f32" else torch.empty(m, n, dtype=tdt, device=DEV)
        run(a_, w, c, flags=flags)
        return c

    first = gemm(a, c0)
    again = gemm(a, c0)
    permuted = gemm(a[perm].contiguous(), c0[perm].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    diff = int((first[perm] != permuted).sum())
    print(f"  permuted rows: {diff} values differ", flush=True)
    assert diff == 0


def test_linear_strided_operands(gpu, oracle, gemm_path):
    """lda > k (a column slice of a wider activation) and ldc > n (writing into a wider buffer)."""
    m, n, k, lda, ldc = 70, 48, 32, 40, 64
    r = np.random.default_rng(3)
    a_full = r.standard_normal((m, lda)).astype(np.float32)
    w = r.standard_normal((n, k)).astype(np.float32)
    c = torch.full((m, ldc), 7.0, device=DEV)
    chronos2.linear(_t(a_full), _t(w), c, m=m, n=n, k=k, lda=lda, ldc=ldc)
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    assert oracle.rel_max_error(got[:, :n], oracle.linear(np.ascontiguousarray(a_full[:, :k]), w)) <= 1e-5
    assert (got[:, n:] == 7.0).all()  # columns past n untouched


@pytest.mark.parametrize("rows,d", [(1, 4), (13, 64), (300, 768)])
def test_rms_norm_matches_oracle(gpu, oracle, rows, d):
    r = np.random.default_rng(rows + d)
    x = (3 * r.standard_normal((rows, d))).astype(np.float32)
    w = r.standard_normal(d).astype(np.float32)
    y = torch.empty(rows, d, device=DEV)
    chronos2.rms_norm(_t(x), _t(w), y, 1e-6)
    torch.cuda.synchronize()
    assert oracle.rel_max_error(y.cpu().numpy(), oracle.rms_norm(x, w, 1e-6)) <= 1e-5


MATRICES = ("time_qkv", "time_o", "group_qkv", "group_o", "wi", "wo")


def _run_layer(x, w, live, group, rows, n, heads, dh, dff, eps, dtype=None):
    d = x.shape[1]
    inner = heads * dh
    xt = _t(x)
    wt = {k: _t(v) for k, v in w.items()}
    code = _lib.JC_F32
    if dtype == "f16x3":  # the weight matrices as fp16 W-operand splits [n, 3k], made on the device
        code = _lib.JC_F16X3
        for k in MATRICES:
            x3 = torch.empty(wt[k].shape[0], 3 * wt[k].shape[1], dtype=torch.float16, device=DEV)
            chronos2.split_f16x3(wt[k], x3, weights=True)
            wt[k] = x3
    elif dtype is not None:  # the weight matrices in the storage type, converted on the device
        code = {torch.bfloat16: _lib.JC_BF16, torch.float16: _lib.JC_F16}[dtype]
        for k in MATRICES:
            lp = torch.empty(wt[k].shape, dtype=dtype, device=DEV)
            chronos2.to_lp(wt[k], lp)
            wt[k] = lp
    gs, ge = chronos2.group_bounds(group)
    table = _t(chronos2.rope_table(n, dh))
    nbytes = chronos2.layer_workspace_bytes(rows, n, d, inner, dff, code)
    ws = torch.empty(nbytes // 4 + 64, device=DEV)
    chronos2.layer(xt, wt, _t(live.reshape(-1).astype(np.int32)), table, _t(gs), _t(ge), ws, rows, n, d, heads, dh,
                   dff, eps, code)
    torch.cuda.synchronize()
    return xt.cpu().numpy()


@pytest.mark.parametrize("rows,n,heads,dh,d,dff,bias", [
    (6, 37, 4, 16, 64, 128, False),
    (6, 37, 4, 16, 64, 128, True),
    (4, 37, 8, 64, 512, 2048, False),    # config 0's layer shape (d_model 512, 8 x 64)
    (3, 130, 12, 64, 768, 3072, False),  # config 4's layer shape (d_model 768, 12 x 64), 130 tokens
])
def test_layer_matches_oracle(gpu, oracle, gemm_path, rows, n, heads, dh, d, dff, bias):
    print(f"case rows={rows} n={n} heads={heads} dh={dh} d={d} dff={dff} bias={bias}", flush=True)
    w = _layer_weights(21 + d, d, heads * dh, dff, bias)
    x = np.random.default_rng(22).standard_normal((rows * n, d)).astype(np.float32)
    live = cases.left_pad_live(23, rows, n, n // 3)
    group = np.sort(np.random.default_rng(24).integers(0, max(1, rows // 2), rows)).astype(np.int32)
    got = _run_layer(x, w, live, group, rows, n, heads, dh, dff, 1e-6)
    exp = oracle.c2_layer(x, w, live, group, rows, n, heads, dh, 1e-6)
    err = oracle.rel_max_error(got, exp)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert err <= TOL


@pytest.mark.parametrize("rows,n,heads,dh,d,dff,bias", [
    (6, 37, 4, 16, 64, 128, True),
    (4, 37, 8, 64, 512, 2048, False),    # config 0's layer shape
    (3, 130, 12, 64, 768, 3072, False),  # config 4's layer shape
])
def test_layer_f16x3_matches_oracle(gpu, oracle, gemm_path, rows, n, heads, dh, d, dff, bias):
    """JC_F16X3: every GEMM on three-term fp16 splits of its operands, fp32 accumulation and outputs,
    held to the fp32 bar (1e-4), at the configs' initialisation (weights N(0, 0.02))."""
    print(f"case f16x3 rows={rows} n={n} heads={heads} dh={dh} d={d} dff={dff} bias={bias}", flush=True)
    w = _layer_weights(41 + d, d, heads * dh, dff, bias)
    r = np.random.default_rng(45)
    for k in MATRICES:
        w[k] = (0.02 * r.standard_normal(w[k].shape)).astype(np.float32)
    x = np.random.default_rng(42).standard_normal((rows * n, d)).astype(np.float32)
    live = cases.left_pad_live(43, rows, n, n // 3)
    group = np.sort(np.random.default_rng(44).integers(0, max(1, rows // 2), rows)).astype(np.int32)
    got = _run_layer(x, w, live, group, rows, n, heads, dh, dff, 1e-6, "f16x3")
    exp = oracle.c2_layer(x, w, live, group, rows, n, heads, dh, 1e-6)
    err = oracle.rel_max_error(got, exp)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert err <= TOL


def _split_reference(v, weights):
    """numpy's round-to-nearest-even float16 of the saturated value, and of what it leaves."""
    v = v.astype(np.float32)
    sat = np.where(np.isnan(v), v, np.clip(v, -65504, 65504)).astype(np.float32)
    hi = sat.astype(np.float16)
    rest = (v - hi.astype(np.float32)).astype(np.float32)
    lo = np.where(np.isnan(rest), rest, np.clip(rest, -65504, 65504)).astype(np.float16)
    return np.concatenate([hi, lo, hi] if weights else [hi, hi, lo], axis=1)


@pytest.mark.parametrize("weights", [False, True])
def test_split_f16x3_is_exact(gpu, weights):
    """jc_split_f16x3 bit for bit against numpy's float16 rounding, with a row stride past k, values
    at fp16's range and past it (saturated), subnormal residues and NaN. hi + lo restores v to 2^-22
    of v plus half fp16's subnormal spacing (2^-25, where lo is subnormal: |v| below about 0.25)."""
    rows, k, ld = 37, 68, 72
    r = np.random.default_rng(9)
    src = (r.standard_normal((rows, ld)) * np.exp(r.uniform(-12, 8, (rows, ld)))).astype(np.float32)
    src[0, :6] = [65504.0, -65504.0, 1e6, -3e5, np.nan, 3.0e-8]
    x = _t(src)
    y = torch.empty(rows, 3 * k, dtype=torch.float16, device=DEV)
    chronos2.split_f16x3(x[:, :k], y, weights=weights)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    exp = _split_reference(src[:, :k], weights)
    np.testing.assert_array_equal(got.view(np.uint16), exp.view(np.uint16))
    hi = got[:, :k].astype(np.float64)
    lo = got[:, k:2 * k] if weights else got[:, 2 * k:]
    v = src[:, :k].astype(np.float64)
    ok = np.isfinite(v) & (np.abs(v) < 60000)
    recon = hi + lo.astype(np.float64)
    assert np.all(np.abs(recon[ok] - v[ok]) <= 2 ** -22 * np.abs(v[ok]) + 2 ** -25)


def test_rms_norm_x3_is_the_split_of_the_norm(gpu):
    """jc_rms_norm_lp with JC_F16X3 writes the A-operand split [hi | hi | lo] of rmsNorm(x): both hi
    copies equal, and hi + lo within 2^-21 of jc_rms_norm's fp32 result plus fp16's subnormal
    spacing (the split's 2^-22 and an ulp of the norm's own rounding)."""
    rows, d = 45, 136
    r = np.random.default_rng(3)
    x = _t((r.standard_normal((rows, d)) * 3).astype(np.float32))
    w = _t((1 + 0.1 * r.standard_normal(d)).astype(np.float32))
    y3 = torch.empty(rows, 3 * d, dtype=torch.float16, device=DEV)
    y = torch.empty(rows, d, device=DEV)
    chronos2.rms_norm_x3(x, w, y3, 1e-6)
    chronos2.rms_norm(x, w, y, 1e-6)
    torch.cuda.synchronize()
    got = y3.cpu().numpy()
    ref = y.cpu().numpy().astype(np.float64)
    np.testing.assert_array_equal(got[:, :d].view(np.uint16), got[:, d:2 * d].view(np.uint16))
    recon = got[:, :d].astype(np.float64) + got[:, 2 * d:].astype(np.float64)
    assert np.all(np.abs(recon - ref) <= 2 ** -21 * np.abs(ref) + 2 ** -24)
    with pytest.raises(JitcastArgumentError):
        chronos2.rms_norm_x3(x, w, torch.empty(rows, 2 * d, dtype=torch.float16, device=DEV), 1e-6)


LP = {"bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.mark.parametrize("dt", sorted(LP))
@pytest.mark.parametrize("m,n,k", [(1, 16, 16), (37, 100, 64), (300, 257, 776), (513, 256, 768),
                                   (20011, 1000, 72)])  # 316 tiles: several per workgroup
@pytest.mark.parametrize("flags,bias,out", [(0, False, "lp"), (chronos2.GEMM_RELU, True, "lp"), (0, True, "f32"),
                                            (chronos2.GEMM_ACCUMULATE, False, "f32"),
                                            (chronos2.GEMM_RELU | chronos2.GEMM_ACCUMULATE, True, "f32")])
def test_linear_lp_matches_oracle(gpu, oracle, gemm_path, m, n, k, flags, bias, out, dt):
    """bf16/fp16 GEMM: exact to fp32-accumulation rounding of the rounded operands (the oracle on
    the same rounded values), then rounded to the output type."""
    print(f"case {dt} m={m} n={n} k={k} flags={flags} bias={bias} out={out}", flush=True)
    r = np.random.default_rng(m + n + k + flags)
    a = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = r.standard_normal(n).astype(np.float32) if bias else None
    c0 = r.standard_normal((m, n)).astype(np.float32)
    at, wt = _t(a).to(LP[dt]), _t(w).to(LP[dt])
    c = _t(c0) if out == "f32" else torch.empty(m, n, dtype=LP[dt], device=DEV)
    chronos2.linear_lp(at, wt, c, bias=_t(b) if bias else None, flags=flags)
    torch.cuda.synchronize()
    exp = _epilogue(oracle.linear(at.float().cpu().numpy(), wt.float().cpu().numpy()), c0, b, flags)
    got = c.float().cpu().numpy()
    tol = 1e-5 if out == "f32" else 2 ** -8  # one rounding to the storage type
    assert oracle.rel_max_error(got, exp) <= tol


@pytest.mark.parametrize("dt", sorted(LP))
def test_linear_lp_strided_operands(gpu, oracle, gemm_path, dt):
    """A, W and C as row slices of wider buffers (lda = 96 > k = 40, ldc = 70 > n = 65)."""
    r = np.random.default_rng(3)
    m, n, k = 300, 65, 40
    abuf = r.standard_normal((m, 96)).astype(np.float32)
    w = (r.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    cbuf = r.standard_normal((m, 70)).astype(np.float32)
    at, wt = _t(abuf).to(LP[dt]), _t(w).to(LP[dt])
    c = _t(cbuf)
    chronos2.linear_lp(at, wt, c, flags=chronos2.GEMM_ACCUMULATE, m=m, n=n, k=k, lda=96, ldc=70)
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    exp = cbuf.copy()
    exp[:, :n] += oracle.linear(np.ascontiguousarray(at.float().cpu().numpy()[:, :k]), wt.float().cpu().numpy())
    assert oracle.rel_max_error(got[:, :n], exp[:, :n]) <= 1e-5
    np.testing.assert_array_equal(got[:, n:], cbuf[:, n:])  # columns past n untouched


@pytest.mark.parametrize("dt", sorted(LP))
def test_rms_norm_lp_and_to_lp(gpu, oracle, dt):
    r = np.random.default_rng(4)
    x = (3 * r.standard_normal((77, 768))).astype(np.float32)
    w = r.standard_normal(768).astype(np.float32)
    y = torch.empty(77, 768, dtype=LP[dt], device=DEV)
    chronos2.rms_norm_lp(_t(x), _t(w), y, 1e-6)
    big = np.array([1e30, -1e30, 7e4, -7e4, 1.5, np.nan, 0.0, -2.5], np.float32)
    z = torch.empty(8, dtype=LP[dt], device=DEV)
    chronos2.to_lp(_t(big), z)
    torch.cuda.synchronize()
    exp = oracle.rms_norm(x, w, 1e-6)
    # one rounding of the fp32 norm (the sums differ in order from the oracle's: at most one ulp of T)
    assert oracle.rel_max_error(y.float().cpu().numpy(), exp) <= 2 ** -8
    zz = z.float().cpu().numpy()
    finite_max = float(torch.finfo(LP[dt]).max)
    assert zz[0] <= finite_max and zz[1] >= -finite_max and np.isfinite(zz[[0, 1, 2, 3]]).all()  # saturated
    assert np.isnan(zz[5]) and zz[4] == 1.5 and zz[7] == -2.5


@pytest.mark.parametrize("dt", sorted(LP))
@pytest.mark.parametrize("rows,n,heads,dh,d,dff", [(6, 37, 4, 16, 64, 128), (3, 260, 12, 64, 768, 3072)])
def test_layer_lp_matches_fp32_oracle(gpu, oracle, gemm_path, rows, n, heads, dh, d, dff, dt):
    """The bf16/fp16 layer against the fp32 oracle on the unrounded weights and inputs, at the
    bf16/fp16 bar (2e-2)."""
    print(f"case {dt} rows={rows} n={n} heads={heads} dh={dh} d={d} dff={dff}", flush=True)
    # the benchmark configurations' initialisation (weights N(0, 0.02), norms 1 +- 0.1, biases 0.1):
    # unscaled Chronos-2 scores then have a std of about 2.5 (with 1/sqrt(in) weights they reach 8,
    # and bf16's 8-bit mantissa alone moves such a softmax by a few percent)
    w = _layer_weights(31 + d, d, heads * dh, dff, True)
    r = np.random.default_rng(35)
    for k in MATRICES:
        w[k] = (0.02 * r.standard_normal(w[k].shape)).astype(np.float32)
    x = np.random.default_rng(32).standard_normal((rows * n, d)).astype(np.float32)
    live = cases.left_pad_live(33, rows, n, n // 3)
    group = np.sort(np.random.default_rng(34).integers(0, max(1, rows // 2), rows)).astype(np.int32)
    got = _run_layer(x, w, live, group, rows, n, heads, dh, dff, 1e-6, LP[dt])
    exp = oracle.c2_layer(x, w, live, group, rows, n, heads, dh, 1e-6)
    err = oracle.rel_max_error(got, exp)
    print(f"  rel err {err:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert err <= 2e-2


def test_layer_rejects_bad_arguments(gpu):
    x = torch.zeros(10, 64, device=DEV)
    with pytest.raises(JitcastArgumentError):
        chronos2.linear(x, torch.zeros(8, 60, device=DEV), torch.zeros(10, 8, device=DEV), k=60)  # k % 16
    with pytest.raises(JitcastArgumentError):
        chronos2.linear(x, torch.zeros(8, 64, device=DEV), torch.zeros(10, 8, device=DEV),
                        flags=chronos2.GEMM_RELU | chronos2.GEMM_SILU)
    with pytest.raises(JitcastArgumentError):
        chronos2.linear(x, torch.zeros(8, 64, device=DEV), torch.zeros(10, 8, device=DEV), flags=chronos2.GEMM_BIAS)
    w = {k: torch.zeros(1, device=DEV) for k in ("time_norm", "time_qkv", "time_o", "group_norm", "group_qkv",
                                                   "group_o", "mlp_norm", "wi", "wo")}
    ws = torch.zeros(1024, device=DEV)
    with pytest.raises(JitcastArgumentError):  # dh past 64
        chronos2.layer(x, w, None, None, None, None, ws, 1, 10, 64, 1, 80, 128, 1e-6)
    with pytest.raises(JitcastArgumentError):  # ACCUMULATE into a bf16 C
        xb = x.to(torch.bfloat16)
        chronos2.linear_lp(xb, torch.zeros(8, 64, dtype=torch.bfloat16, device=DEV),
                           torch.zeros(10, 8, dtype=torch.bfloat16, device=DEV), flags=chronos2.GEMM_ACCUMULATE)
    with pytest.raises(JitcastArgumentError):  # JC_GEMM_BIAS with no bias: rejected before any launch
        chronos2.linear_lp(x.to(torch.bfloat16), torch.zeros(8, 64, dtype=torch.bfloat16, device=DEV),
                           torch.zeros(10, 8, device=DEV), flags=chronos2.GEMM_BIAS)
