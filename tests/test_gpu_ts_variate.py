"""GPU parity of Timestral variate attention (BlockLayout.variateAllowed, 1/sqrt(dh) scale,
optional sigmoid gate) against the C oracle, through the C ABI. Bar: max relative error <= 1e-4."""
import numpy as np
import pytest
import torch

from jitcast_amd import chronos2, rng, timestral
from tests import cases

pytestmark = pytest.mark.gpu
TOL_F32 = 1e-4


def _roles(seed, rows):
    """TARGET 0 / PAST 1 / KNOWN 2 (BlockInput.java:35-37), seeded."""
    return np.floor(rng.uniform(rng.stream_seed(seed, 6), rows) * 3).astype(np.int32)


def _run(qkv, kv, group, role, cov, gate, rows, enc, n, heads, dh, d):
    dev = torch.device("cuda:0")
    s, e = chronos2.group_bounds(group)

    def i32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.int32).reshape(-1)).to(dev)

    out = torch.full((rows * n, d), float("nan"), device=dev)
    g = torch.from_numpy(gate).to(dev) if gate is not None else None
    timestral.variate_attention(torch.from_numpy(qkv).to(dev), out, i32(kv), i32(s), i32(e), i32(role), cov, g, rows,
                                enc, n, heads, dh, d)
    torch.cuda.synchronize()
    return out.cpu().numpy()


CASES = [
    # rows, enc, h, heads, dh, d, group sizes lo..hi, covariates, valid probability, gate
    (37, 6, 2, 2, 64, 128, 1, 8, 0, 0.7, False),
    (64, 5, 3, 3, 64, 192, 1, 64, 1, 0.8, True),
    (100, 4, 1, 2, 64, 128, 100, 100, 1, 0.9, False),  # one group larger than 64 rows
    (45, 4, 2, 2, 32, 72, 1, 1, 0, 0.5, True),  # every row its own group
    (50, 3, 2, 4, 16, 64, 5, 5, 1, 0.7, False),
    (33, 2, 2, 2, 24, 48, 3, 20, 1, 0.6, True),  # dh not a multiple of 16
    (20, 3, 1, 1, 128, 128, 20, 20, 1, 0.6, True),  # 128-wide heads
    (17, 2, 0, 2, 48, 96, 17, 17, 0, 1.0, False),
    (40, 0, 3, 2, 64, 128, 2, 9, 1, 1.0, False),  # decoder slots only
    (96, 4, 2, 4, 64, 256, 3, 3, 1, 0.8, True),  # a target and 2 covariates per group: packs of 5 groups
    # one-row groups (univariate series) take the streaming path per 16-row tile
    (80, 7, 2, 12, 64, 768, 1, 1, 1, 0.6, True),
    (21, 3, 1, 2, 128, 256, 1, 1, 0, 0.7, False),
    (19, 2, 2, 3, 24, 72, 1, 1, 0, 0.5, True),
    (35, 3, 1, 2, 48, 96, 1, 1, 1, 0.8, False),
    (70, 3, 1, 2, 64, 128, 1, 2, 0, 0.7, True),  # tiles of singletons beside mixed tiles
]


@pytest.mark.parametrize("rows,enc,h,heads,dh,d,lo,hi,cov,p,gate", CASES)
def test_fp32_matches_oracle(gpu, oracle, rows, enc, h, heads, dh, d, lo, hi, cov, p, gate):
    print(f"case rows={rows} enc={enc} h={h} heads={heads} dh={dh} groups {lo}..{hi} cov={cov} gate={gate}",
          flush=True)
    n = enc + h
    qkv = cases.qkv(107, rows * n, d)
    kv = cases.random_live(107, rows, max(enc, 1), p)[:, :enc].copy()
    group = cases.group_sizes(107, rows, lo, hi)
    role = _roles(107, rows) if cov else np.zeros(rows, np.int32)
    g = cases.qkv(108, rows * n, d)[:, :d].copy() if gate else None
    got = _run(qkv, kv, group, role, cov, g, rows, enc, n, heads, dh, d)[:, : heads * dh]
    exp = oracle.ts_variate_attention(qkv, kv, group, role, cov, rows, enc, n, heads, dh, d)
    if g is not None:
        exp = oracle.ts_gate(exp, g)
    exp = exp[:, : heads * dh]
    assert np.isfinite(got).all()
    err = oracle.rel_max_error(got, exp)
    print(f"  rel err {err:.3e}", flush=True)
    assert err <= TOL_F32


def test_known_rows_never_read_other_rows(gpu, oracle):
    """A group of known-covariate rows plus one target: perturbing the target's k/v leaves every
    known row's output bit for bit (BlockLayout.java:236-238)."""
    rows, enc, h, heads, dh, d = 6, 3, 1, 2, 64, 128
    n = enc + h
    qkv = cases.qkv(109, rows * n, d)
    kv = np.ones((rows, enc), np.int32)
    group = np.zeros(rows, np.int32)
    role = np.array([0, 2, 2, 1, 2, 0], np.int32)
    base = _run(qkv, kv, group, role, 1, None, rows, enc, n, heads, dh, d).reshape(rows, n, d)
    p = qkv.copy().reshape(rows, n, 3 * d)
    p[[0, 5], :, d:] += 2.0
    pert = _run(p.reshape(rows * n, -1), kv, group, role, 1, None, rows, enc, n, heads, dh, d).reshape(rows, n, d)
    np.testing.assert_array_equal(pert[[1, 2, 4]], base[[1, 2, 4]])
    np.testing.assert_array_equal(pert[3], base[3])  # a PAST covariate never reads targets either
    assert np.abs(pert[0] - base[0]).max() > 1e-3


LP = {"bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.mark.parametrize("dt", sorted(LP))
@pytest.mark.parametrize("rows,enc,h,heads,dh,d,lo,hi,cov,p,gate", CASES)
def test_lowp_matches_oracle(gpu, oracle, dt, rows, enc, h, heads, dh, d, lo, hi, cov, p, gate):
    """bf16 / fp16 storage of q|k|v, the gate and out, fp32 arithmetic: against the oracle on the same
    rounded inputs within 2^-8 (bf16) / 2^-11 (fp16), and on the unrounded fp32 inputs within 2e-2."""
    print(f"case {dt} rows={rows} enc={enc} h={h} heads={heads} dh={dh} groups {lo}..{hi} cov={cov} gate={gate}",
          flush=True)
    dev = torch.device("cuda:0")
    n = enc + h
    qkv = cases.qkv(107, rows * n, d)
    kv = cases.random_live(107, rows, max(enc, 1), p)[:, :enc].copy()
    group = cases.group_sizes(107, rows, lo, hi)
    role = _roles(107, rows) if cov else np.zeros(rows, np.int32)
    g = cases.qkv(108, rows * n, d)[:, :d].copy() if gate else None
    s, e = chronos2.group_bounds(group)

    def i32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.int32).reshape(-1)).to(dev)

    q = torch.from_numpy(qkv).to(dev).to(LP[dt])
    gt = torch.from_numpy(g).to(dev).to(LP[dt]) if g is not None else None
    out = torch.full((rows * n, d), float("nan"), dtype=LP[dt], device=dev)
    timestral.variate_attention(q, out, i32(kv), i32(s), i32(e), i32(role), cov, gt, rows, enc, n, heads, dh, d)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()[:, : heads * dh]
    assert np.isfinite(got).all()

    def expect(qkv_in, g_in):
        x = oracle.ts_variate_attention(qkv_in, kv, group, role, cov, rows, enc, n, heads, dh, d)
        return (oracle.ts_gate(x, g_in) if g_in is not None else x)[:, : heads * dh]

    exp_r = expect(q.float().cpu().numpy(), gt.float().cpu().numpy() if gt is not None else None)
    exp = expect(qkv, g)
    err_r, err = oracle.rel_max_error(got, exp_r), oracle.rel_max_error(got, exp)
    print(f"  rel err {err_r:.3e} on the rounded inputs, {err:.3e} against fp32", flush=True)
    assert err_r <= (2.0 ** -8 if dt == "bf16" else 2.0 ** -11)
    assert err <= 2e-2


def test_univariate_rows_output_their_own_v(gpu):
    """A one-row group's only key is the row itself (always allowed, BlockLayout.java:228-230): its
    softmax weight is 1, so the output is its own v bit for bit, whatever the key validity."""
    rows, enc, h, heads, dh, d = 40, 5, 2, 12, 64, 768
    n = enc + h
    qkv = cases.qkv(111, rows * n, d)
    kv = cases.random_live(111, rows, enc, 0.5)
    group = np.arange(rows, dtype=np.int32)
    got = _run(qkv, kv, group, np.zeros(rows, np.int32), 0, None, rows, enc, n, heads, dh, d)
    np.testing.assert_array_equal(got, qkv[:, 2 * d:])
