"""GPU parity of the fused Chronos-2 time attention against the C oracle (through the C ABI).

Bar: max relative error (the reference's metric) <= 1e-4 for fp32 and <= 2e-2 for bf16/fp16 (qkv
rounded to the storage type, compared with the fp32 oracle on the unrounded qkv).
"""
import numpy as np
import pytest
import torch

from jitcast_amd import JitcastArgumentError, chronos2
from tests import brute, cases

pytestmark = pytest.mark.gpu
TOL_F32 = 1e-4
TOL_LP = 2e-2
LP_DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _run(qkv, live, rows, n, heads, dh, inner, table=True, dtype=torch.float32):
    dev = torch.device("cuda:0")
    q = torch.from_numpy(qkv).to(dev).to(dtype)
    out = torch.full((rows * n, inner), float("nan"), dtype=dtype, device=dev)
    tab = torch.from_numpy(chronos2.rope_table(n, dh)).to(dev) if table else None
    chronos2.time_attention(q, out, torch.from_numpy(np.ascontiguousarray(live.reshape(-1), np.int32)).to(dev),
                            rows, n, heads, dh, inner, tab)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    # rows, n, heads, dh, inner, live kind
    (2, 37, 2, 64, 128, "pad"),
    (1, 1, 1, 64, 64, "all"),
    (2, 2, 1, 64, 64, "all"),
    (3, 31, 2, 64, 128, "random"),
    (3, 32, 2, 64, 128, "random"),
    (3, 33, 2, 64, 128, "pad"),
    (2, 129, 3, 64, 192, "random"),
    (2, 200, 2, 64, 136, "pad"),
    (2, 77, 3, 32, 96, "pad"),
    (2, 50, 2, 48, 100, "random"),
    (2, 45, 4, 16, 64, "pad"),
    (1, 600, 1, 64, 64, "pad"),
    (2, 257, 2, 64, 128, "random"),
    (1, 129, 2, 64, 128, "all"),
]


def _live(kind, seed, rows, n):
    if kind == "pad":
        return cases.left_pad_live(seed, rows, n, n // 2)
    if kind == "random":
        return cases.random_live(seed, rows, n, 0.5)
    return np.ones((rows, n), np.int32)


@pytest.mark.parametrize("rows,n,heads,dh,inner,kind", CASES)
def test_fp32_matches_oracle(gpu, oracle, rows, n, heads, dh, inner, kind):
    print(f"case rows={rows} n={n} heads={heads} dh={dh} inner={inner} {kind}", flush=True)
    qkv = cases.qkv(23, rows * n, inner)
    live = _live(kind, 23, rows, n)
    got = _run(qkv, live, rows, n, heads, dh, inner)
    exp = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner)
    # columns past heads*dh are not attention outputs: the kernel leaves them untouched
    got, exp = got[:, : heads * dh], exp[:, : heads * dh]
    assert np.isfinite(got).all()
    assert oracle.rel_max_error(got, exp) <= TOL_F32


LP_CASES = [c for c in CASES if c[3] % 16 == 0 and c[4] % 8 == 0] + [
    (2, 513, 2, 64, 128, "pad"),
    (1, 1030, 1, 64, 64, "random"),
    (3, 300, 2, 64, 136, "random"),
    (1, 257, 1, 64, 64, "pad"),
    (2, 512, 3, 64, 192, "random"),
    (3, 133, 2, 64, 128, "pad"),  # 5 query tiles: 5 waves per item in the short-row persistent kernel
    (2, 160, 2, 64, 128, "random"),
    (2, 65, 2, 64, 128, "random"),  # the shortest row the short-row kernel takes: 2 blocks, 3 tiles
    (3, 96, 2, 64, 128, "pad"),
    (2, 100, 3, 64, 192, "all"),  # 4 tiles
    (2, 128, 2, 64, 136, "random"),
    (1, 64, 2, 64, 128, "random"),  # one block: the streaming kernel
]


@pytest.mark.parametrize("dt", sorted(LP_DTYPES))
@pytest.mark.parametrize("rows,n,heads,dh,inner,kind", LP_CASES)
def test_lowp_matches_oracle(gpu, oracle, rows, n, heads, dh, inner, kind, dt, lp_kernel):
    # (a shape the chosen kernel does not take runs on the streaming kernel: the fallback is tested too)
    print(f"case {dt} {lp_kernel} rows={rows} n={n} heads={heads} dh={dh} inner={inner} {kind}", flush=True)
    qkv = cases.qkv(53, rows * n, inner, std=0.554)
    live = _live(kind, 53, rows, n)
    got = _run(qkv, live, rows, n, heads, dh, inner, dtype=LP_DTYPES[dt])[:, : heads * dh]
    assert np.isfinite(got).all()
    exp = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner)[:, : heads * dh]
    err = oracle.rel_max_error(got, exp)
    # the kernel's own error: the oracle on the same rounded inputs
    rounded = torch.from_numpy(qkv).to(LP_DTYPES[dt]).float().numpy()
    own = oracle.rel_max_error(got, oracle.c2_time_attention(rounded, live, rows, n, heads, dh, inner)[:, : heads * dh])
    print(f"  rel err {err:.3e} (vs rounded inputs {own:.3e})", flush=True)
    assert err <= TOL_LP
    assert own <= TOL_LP / 2


@pytest.mark.parametrize("dt", sorted(LP_DTYPES))
def test_lowp_one_live_key_returns_its_value(gpu, dt):
    rows, n, heads, dh, inner = 2, 70, 2, 64, 128
    qkv = cases.qkv(31, rows * n, inner)
    live = np.zeros((rows, n), np.int32)
    live[0, 3] = 1
    live[1, 69] = 1
    got = _run(qkv, live, rows, n, heads, dh, inner, dtype=LP_DTYPES[dt]).reshape(rows, n, inner)
    v = torch.from_numpy(qkv).to(LP_DTYPES[dt]).float().numpy().reshape(rows, n, 3 * inner)[:, :, 2 * inner:]
    # softmax of one key is exactly 1: the output is that key's v, bit for bit in the storage type
    np.testing.assert_array_equal(got[0], np.broadcast_to(v[0, 3], (n, inner)))
    np.testing.assert_array_equal(got[1], np.broadcast_to(v[1, 69], (n, inner)))


@pytest.mark.parametrize("dt", sorted(LP_DTYPES))
def test_lowp_no_live_key_gives_zeros(gpu, dt):
    rows, n, heads, dh, inner = 3, 40, 2, 64, 128
    qkv = cases.qkv(29, rows * n, inner)
    live = cases.left_pad_live(29, rows, n, 10)
    live[1] = 0
    got = _run(qkv, live, rows, n, heads, dh, inner, dtype=LP_DTYPES[dt]).reshape(rows, n, inner)
    assert not np.any(got[1])
    assert np.isfinite(got).all()


def _lowp_operand_model(qkv_rounded, live, rows, n, heads, dh, inner, tdtype):
    """float64 attention over the operands the MFMAs actually see: q rotated, scaled by log2(e) and
    rounded to the storage type; k rotated and rounded; v as stored. Isolates the kernel's softmax
    logic from operand rounding (which at large score scales dominates any bf16 kernel's error)."""
    q, k, v = brute.split_qkv(qkv_rounded, rows, n, heads, dh, inner)
    pos = np.broadcast_to(np.arange(n), (rows, n))
    inv = brute.inv_freq(dh)
    l2e = np.float32(1.4426950408889634)

    def rnd(x):
        return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(tdtype).double().numpy()

    qr = rnd(brute.rope_float(q, pos, inv) * l2e).transpose(0, 2, 1, 3)
    kr = rnd(brute.rope_float(k, pos, inv)).transpose(0, 2, 1, 3)
    s = qr @ kr.transpose(0, 1, 3, 2)  # log2 units
    s = np.where(live[:, None, None, :] == 1, s, -np.inf)
    p = np.exp2(s - s.max(-1, keepdims=True))
    o = (p / p.sum(-1, keepdims=True)) @ v.astype(np.float64).transpose(0, 2, 1, 3)
    return o.transpose(0, 2, 1, 3).reshape(rows * n, heads * dh)


@pytest.mark.parametrize("dt", sorted(LP_DTYPES))
@pytest.mark.parametrize("std,n", [(2.5, 300), (6.0, 129), (0.05, 200)])
def test_lowp_extreme_score_scales(gpu, oracle, dt, std, n):
    """Large scores move the block max by tens of log2 units between blocks (the rescaling slow
    path on most blocks); tiny scores keep every block on the fast path. Checked against the
    float64 model of the rounded MFMA operands."""
    rows, heads, dh, inner = 2, 2, 64, 128
    qkv = cases.qkv(59, rows * n, inner, std=std)
    live = cases.left_pad_live(59, rows, n, n // 3)
    got = _run(qkv, live, rows, n, heads, dh, inner, dtype=LP_DTYPES[dt])[:, : heads * dh]
    assert np.isfinite(got).all()
    rounded = torch.from_numpy(qkv).to(LP_DTYPES[dt]).float().numpy()
    exp = _lowp_operand_model(rounded, live, rows, n, heads, dh, inner, LP_DTYPES[dt])
    err = oracle.rel_max_error(got, exp)
    print(f"  std {std}: rel err vs the operand model {err:.3e}", flush=True)
    assert err <= TOL_LP / 2


def test_bf16_config1_shape_subset_matches_oracle(gpu, oracle, lp_kernel):
    """Config 1-bf16: the config-1 inputs (12 series) with qkv rounded to bf16, against the fp32 oracle."""
    from jitcast_amd import synthetic

    case = synthetic.c2_time_config1(rows=12, device="cuda")
    q16 = case.qkv.to(torch.bfloat16)
    out = torch.empty(case.rows * case.n, case.inner, device="cuda", dtype=torch.bfloat16)
    chronos2.time_attention(q16, out, case.live, case.rows, case.n, case.heads, case.dh, case.inner, case.table)
    torch.cuda.synchronize()
    exp = oracle.c2_time_attention(case.qkv.cpu().numpy(), case.live.cpu().numpy(), case.rows, case.n, case.heads,
                                   case.dh, case.inner)
    err = oracle.rel_max_error(out.float().cpu().numpy(), exp)
    print(f"config-1 bf16 subset ({lp_kernel}) rel err {err:.3e}", flush=True)
    assert err <= TOL_LP


@pytest.mark.parametrize("n", [40, 129, 133])
def test_fp32_no_live_key_gives_zeros(gpu, oracle, n):
    rows, heads, dh, inner = 3, 2, 64, 128
    qkv = cases.qkv(29, rows * n, inner)
    live = cases.left_pad_live(29, rows, n, 10)
    live[1] = 0
    got = _run(qkv, live, rows, n, heads, dh, inner)
    assert not np.any(got.reshape(rows, n, inner)[1])
    exp = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner)
    assert oracle.rel_max_error(got, exp) <= TOL_F32


@pytest.mark.parametrize("n", [70, 129, 133])
def test_fp32_one_live_key_returns_its_value(gpu, n):
    rows, heads, dh, inner = 2, 2, 64, 128
    qkv = cases.qkv(31, rows * n, inner)
    live = np.zeros((rows, n), np.int32)
    live[0, 3] = 1
    live[1, n - 1] = 1
    got = _run(qkv, live, rows, n, heads, dh, inner).reshape(rows, n, inner)
    v = qkv.reshape(rows, n, 3 * inner)[:, :, 2 * inner:]
    np.testing.assert_allclose(got[0], np.broadcast_to(v[0, 3], (n, inner)), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(got[1], np.broadcast_to(v[1, n - 1], (n, inner)), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("n,kind", [(129, "pad"), (257, "random"), (513, "pad")])
def test_fp32_folded_last_query(gpu, oracle, n, kind):
    """Rows of 128k + 1 tokens: the last query ([REG]) is computed by the last full workgroup on VALU
    instead of a workgroup of its own. Its output is checked on its own, per head, besides the whole."""
    rows, heads, dh, inner = 3, 3, 64, 200
    print(f"case folded n={n} {kind}", flush=True)
    qkv = cases.qkv(41, rows * n, inner)
    live = _live(kind, 41, rows, n)
    got = _run(qkv, live, rows, n, heads, dh, inner).reshape(rows, n, inner)
    exp = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner).reshape(rows, n, inner)
    assert oracle.rel_max_error(got[:, :, : heads * dh], exp[:, :, : heads * dh]) <= TOL_F32
    for h in range(heads):
        sl = np.s_[:, n - 1, h * dh:(h + 1) * dh]
        assert oracle.rel_max_error(got[sl], exp[sl]) <= TOL_F32, h
    assert np.isnan(got[:, :, heads * dh:]).all(), "columns past heads * dh are not written"


@pytest.mark.parametrize("n,kind,table", [(130, "pad", True), (133, "random", True), (136, "all", True),
                                          (261, "pad", True), (133, "pad", False), (137, "pad", True),
                                          (144, "random", True), (145, "pad", True), (130, "random", False),
                                          (133, "dead", True)])
def test_fp32_tail_queries(gpu, oracle, n, kind, table):
    """Rows of 128k + R tokens (the forecasts' 128 patches + [REG] + 4 future patches give R = 5):
    with 2 <= R <= 16 the main kernel runs the first 128k queries and a kernel of its own the R tail
    queries (R = 17 keeps a fifth workgroup). Against the oracle, the tail rows checked on their own
    per head; "dead": one row without live keys, whose outputs are zeros."""
    rows, heads, dh, inner = 3, 3, 64, 200
    print(f"case tail queries n={n} {kind} table={table}", flush=True)
    qkv = cases.qkv(43, rows * n, inner)
    live = _live("pad" if kind == "dead" else kind, 43, rows, n)
    if kind == "dead":
        live[1] = 0
    got = _run(qkv, live, rows, n, heads, dh, inner, table=table).reshape(rows, n, inner)
    if table:
        exp = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner).reshape(rows, n, inner)
    else:  # qkv taken as already rotated: plain attention over the live keys, in float64
        q, k, v = brute.split_qkv(qkv, rows, n, heads, dh, inner)
        sc = np.einsum("rqhe,rkhe->rhqk", q.astype(np.float64), k.astype(np.float64))
        sc = np.where(live[:, None, None, :] == 1, sc, -np.inf)
        pr = np.exp(sc - sc.max(-1, keepdims=True))
        o = np.einsum("rhqk,rkhe->rqhe", pr / pr.sum(-1, keepdims=True), v.astype(np.float64))
        exp = np.full((rows, n, inner), np.nan)
        exp[:, :, : heads * dh] = o.reshape(rows, n, heads * dh)
    assert oracle.rel_max_error(got[:, :, : heads * dh], exp[:, :, : heads * dh]) <= TOL_F32
    tail = n % 128
    for h in range(heads):
        sl = np.s_[:, n - tail:, h * dh:(h + 1) * dh]
        assert oracle.rel_max_error(got[sl], exp[sl]) <= TOL_F32, h
    if kind == "dead":
        assert not np.any(got[1, :, : heads * dh])
    assert np.isnan(got[:, :, heads * dh:]).all(), "columns past heads * dh are not written"


@pytest.mark.parametrize("n", [33, 161, 513])
@pytest.mark.parametrize("pattern", ["last dead", "only last", "all", "pad"])
def test_fp32_last_key(gpu, oracle, n, pattern):
    """Rows of 32k + 1 tokens: key n - 1 is not staged as a block of its own but added on VALU after
    the block loop (with the folded query too at n = 128k + 1). Checked with that key dead among live
    ones, as the only live key, and with every key or a left-padded row live."""
    rows, heads, dh, inner = 3, 2, 64, 136
    print(f"case last key n={n} {pattern}", flush=True)
    qkv = cases.qkv(43, rows * n, inner)
    live = cases.left_pad_live(43, rows, n, n // 2) if pattern == "pad" else np.ones((rows, n), np.int32)
    if pattern == "last dead":
        live[:, n - 1] = 0
    elif pattern == "only last":
        live[:] = 0
        live[:, n - 1] = 1
    got = _run(qkv, live, rows, n, heads, dh, inner)[:, : heads * dh]
    exp = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner)[:, : heads * dh]
    assert oracle.rel_max_error(got, exp) <= TOL_F32
    if pattern == "only last":
        v = qkv.reshape(rows, n, 3 * inner)[:, n - 1, 2 * inner:2 * inner + heads * dh]
        np.testing.assert_allclose(got.reshape(rows, n, -1), np.broadcast_to(v[:, None], (rows, n, heads * dh)),
                                   rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("n", [65, 129])
def test_fp32_without_table_is_plain_attention(gpu, n):
    """rope_table NULL: qkv is taken as already rotated (the reference's separate rope task ran)."""
    rows, heads, dh, inner = 2, 2, 64, 128
    qkv = cases.qkv(37, rows * n, inner)
    live = cases.left_pad_live(37, rows, n, 30)
    got = _run(qkv, live, rows, n, heads, dh, inner, table=False)
    q, k, v = brute.split_qkv(qkv, rows, n, heads, dh, inner)
    s = np.einsum("rqhe,rkhe->rhqk", q.astype(np.float64), k.astype(np.float64))
    s = np.where(live[:, None, None, :] == 1, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    o = np.einsum("rhqk,rkhe->rqhe", p / p.sum(-1, keepdims=True), v.astype(np.float64))
    from oracle.oracle import rel_max_error
    assert rel_max_error(got, o.reshape(rows * n, inner)) <= TOL_F32


def test_config1_shape_subset_matches_oracle(gpu, oracle):
    """The config-1 shape (L=513, 12x64, d 768, pads U{0..256}) on 12 series generated like the bench."""
    from jitcast_amd import synthetic

    case = synthetic.c2_time_config1(rows=12, device="cuda")
    out = torch.empty(case.rows * case.n, case.inner, device="cuda")
    chronos2.time_attention(case.qkv, out, case.live, case.rows, case.n, case.heads, case.dh, case.inner, case.table)
    torch.cuda.synchronize()
    exp = oracle.c2_time_attention(case.qkv.cpu().numpy(), case.live.cpu().numpy(), case.rows, case.n, case.heads,
                                   case.dh, case.inner)
    err = oracle.rel_max_error(out.cpu().numpy(), exp)
    print(f"config-1 subset rel err {err:.3e}", flush=True)
    assert err <= TOL_F32


def test_rejects_bad_shapes(gpu):
    dev = torch.device("cuda:0")
    q = torch.zeros(4 * 3 * 64, device=dev)
    o = torch.zeros(4 * 64, device=dev)
    lv = torch.ones(4, dtype=torch.int32, device=dev)
    with pytest.raises(JitcastArgumentError, match="head width"):
        chronos2.time_attention(q, o, lv, 1, 4, 1, 12, 64)
    with pytest.raises(JitcastArgumentError, match="inner"):
        chronos2.time_attention(q, o, lv, 1, 4, 2, 64, 64)


@pytest.mark.parametrize("dt", sorted(LP_DTYPES))
@pytest.mark.parametrize("table", [True, False])
@pytest.mark.parametrize("n", [513, 133])
def test_lowp_many_items_per_workgroup(gpu, oracle, dt, table, n, monkeypatch):
    """The persistent kernels walk several (row, head) items per workgroup and stream their blocks
    back to back. 300 rows x 12 heads: at n = 513 every workgroup gets 12 items of different lengths;
    at n = 133 (the short-row kernel) 14 or 15 items split over the workgroup's two halves, so one
    half idles through the last item's steps where the count is odd. Among the rows: one without
    live keys (zeros), one whose only live key is the last token, rows with gaps and left-padded
    rows. Without a table the kernel takes q and k as already rotated."""
    monkeypatch.setenv("JITCAST_HIP_LP_KERNEL", "persist")
    rows, heads, dh = 300, 12, 64
    inner = heads * dh
    print(f"case {dt} persist many items table={table} rows={rows} n={n}", flush=True)
    qkv = cases.qkv(61, rows * n, inner, std=0.554)
    live = cases.left_pad_live(61, rows, n, 256 if n > 256 else n // 2)
    gaps = cases.random_live(61, rows, n, 0.7)
    live[::3] = gaps[::3]
    live[:, n - 1] = 1
    live[5] = 0
    live[7] = 0
    live[7, n - 1] = 1
    live[11, :64] = 1
    live[11, 64:n - 1] = 0
    got = _run(qkv, live, rows, n, heads, dh, inner, table=table, dtype=LP_DTYPES[dt])
    assert np.isfinite(got).all()
    assert not np.any(got.reshape(rows, n, inner)[5])
    rounded = torch.from_numpy(qkv).to(LP_DTYPES[dt]).float().numpy()
    if table:
        exp = oracle.c2_time_attention(rounded, live, rows, n, heads, dh, inner)
        err = oracle.rel_max_error(got, exp)
    else:
        # rows of the first and the last item of every workgroup, and the special rows
        pick = np.r_[0:16, 5, 7, 11, 280:300]
        exp = _plain_attention(rounded, live, pick, n, heads, dh, inner)
        err = oracle.rel_max_error(got.reshape(rows, n, inner)[pick].reshape(-1, inner), exp)
    print(f"  rel err vs the reference on the rounded inputs {err:.3e}", flush=True)
    assert err <= TOL_LP / 2


def _plain_attention(qkv, live, pick, n, heads, dh, inner):
    """float64 masked attention without RoPE or scale on the rows `pick` (torch on the CPU)."""
    x = torch.from_numpy(qkv).double().reshape(-1, n, 3 * inner)[torch.from_numpy(np.asarray(pick))]
    q, k, v = (x[:, :, i * inner:(i + 1) * inner].reshape(len(pick), n, heads, dh).transpose(1, 2).contiguous()
               for i in range(3))
    s = torch.matmul(q, k.transpose(-1, -2).contiguous())
    m = torch.from_numpy(live[pick] == 1)[:, None, None, :]
    s = s.masked_fill(~m, float("-inf"))
    p = torch.softmax(s, -1).nan_to_num(0.0)
    o = torch.matmul(p, v).transpose(1, 2).reshape(len(pick) * n, inner)
    return o.numpy()
