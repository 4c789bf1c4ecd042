"""GPU parity of the fused Timestral time attention (RoPE at pos, BlockLayout.timeAllowed mask,
1/sqrt(dh) scale, optional sigmoid gate) against the C oracle, through the C ABI.

Bar: max relative error <= 1e-4 for fp32, <= 2e-2 for bf16/fp16 (qkv and gate rounded to the
storage type, compared with the fp32 oracle on the unrounded inputs).
"""
import numpy as np
import pytest
import torch

from jitcast_amd import JitcastArgumentError, timestral
from tests import cases

pytestmark = pytest.mark.gpu
TOL_F32 = 1e-4
TOL_LP = 2e-2
DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def _run(qkv, kv, known, position, gate, rows, enc, ll, n, heads, dh, d, rope_dim, dtype=torch.float32,
         with_table=True):
    dev = torch.device("cuda:0")

    def i32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.int32).reshape(-1)).to(dev)

    q = torch.from_numpy(qkv).to(dev).to(dtype)
    out = torch.full((rows * n, d), float("nan"), dtype=dtype, device=dev)
    g = torch.from_numpy(gate).to(dev).to(dtype) if gate is not None else None
    tab = torch.from_numpy(timestral.rope_table(enc, n, dh, rope_dim)).to(dev) if with_table else None
    timestral.time_attention(q, out, i32(kv), i32(known), i32(position + enc), tab, g, rows, enc, ll, n, heads, dh, d)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _expected(oracle, qkv, kv, known, position, gate, rows, enc, ll, n, heads, dh, d, rope_dim):
    exp = oracle.ts_time_attention(qkv, kv, known, position, rows, enc, ll, n, heads, dh, d, rope_dim)
    if gate is not None:
        exp = oracle.ts_gate(exp, gate)
    return exp


CASES = [
    # rows, enc, ll, h, heads, dh, d, rope_dim, known_frac, gate
    (3, 20, 20, 4, 2, 64, 128, 32, 0.0, False),
    (4, 50, 40, 4, 2, 64, 136, 32, 0.5, True),
    (2, 200, 200, 0, 2, 64, 128, 32, 0.0, False),
    (2, 129, 129, 3, 3, 32, 96, 16, 1.0, True),
    (2, 70, 64, 6, 2, 128, 256, 64, 0.3, True),
    (2, 37, 37, 3, 1, 48, 48, 24, 0.0, False),
    (2, 45, 45, 2, 2, 16, 40, 8, 0.5, False),
    (1, 600, 600, 8, 1, 64, 64, 32, 0.0, True),
    (3, 64, 64, 0, 2, 64, 128, 32, 0.0, False),
    (2, 136, 130, 4, 2, 64, 128, 32, 0.3, True),  # 140 tokens: 5 query tiles
]


def _inputs(seed, rows, enc, ll, h, d, known_frac, gate):
    n = enc + h
    qkv = cases.qkv(seed, rows * n, d, std=0.6)
    kv, known, position = cases.ts_layout(seed, rows, enc, ll, h, known_frac)
    g = cases.qkv(seed + 1, rows * n, d)[:, :d].copy() if gate else None
    return n, qkv, kv, known, position, g


@pytest.mark.parametrize("rows,enc,ll,h,heads,dh,d,rope_dim,known_frac,gate", CASES)
def test_fp32_matches_oracle(gpu, oracle, rows, enc, ll, h, heads, dh, d, rope_dim, known_frac, gate):
    print(f"case fp32 rows={rows} enc={enc} ll={ll} h={h} heads={heads} dh={dh} known={known_frac} gate={gate}",
          flush=True)
    n, qkv, kv, known, position, g = _inputs(83, rows, enc, ll, h, d, known_frac, gate)
    got = _run(qkv, kv, known, position, g, rows, enc, ll, n, heads, dh, d, rope_dim)[:, : heads * dh]
    exp = _expected(oracle, qkv, kv, known, position, g, rows, enc, ll, n, heads, dh, d, rope_dim)[:, : heads * dh]
    assert np.isfinite(got).all()
    err = oracle.rel_max_error(got, exp)
    print(f"  rel err {err:.3e}", flush=True)
    assert err <= TOL_F32


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("rows,enc,ll,h,heads,dh,d,rope_dim,known_frac,gate", [c for c in CASES if c[5] % 16 == 0])
def test_lowp_matches_oracle(gpu, oracle, rows, enc, ll, h, heads, dh, d, rope_dim, known_frac, gate, dt, lp_kernel):
    # (a shape the chosen kernel does not take runs on the streaming kernel: the fallback is tested too)
    print(f"case {dt} {lp_kernel} rows={rows} enc={enc} ll={ll} h={h} heads={heads} dh={dh} known={known_frac} gate={gate}",
          flush=True)
    n, qkv, kv, known, position, g = _inputs(89, rows, enc, ll, h, d, known_frac, gate)
    got = _run(qkv, kv, known, position, g, rows, enc, ll, n, heads, dh, d, rope_dim, DTYPES[dt])[:, : heads * dh]
    exp = _expected(oracle, qkv, kv, known, position, g, rows, enc, ll, n, heads, dh, d, rope_dim)[:, : heads * dh]
    assert np.isfinite(got).all()
    err = oracle.rel_max_error(got, exp)
    print(f"  rel err {err:.3e}", flush=True)
    assert err <= TOL_LP


def test_fp32_without_table_is_plain_masked_attention(gpu, oracle):
    """rope_table NULL: q and k are taken as already rotated (rope_dim with a zero table is the
    identity, which the oracle computes when every position is 0)."""
    rows, enc, ll, h, heads, dh, d = 2, 40, 40, 3, 2, 64, 128
    n, qkv, kv, known, position, _ = _inputs(97, rows, enc, ll, h, d, 0.5, False)
    got = _run(qkv, kv, known, position, None, rows, enc, ll, n, heads, dh, d, 32, with_table=False)
    exp = oracle.ts_time_attention(qkv, kv, known, np.zeros_like(position), rows, enc, ll, n, heads, dh, d, 32)
    assert oracle.rel_max_error(got[:, : heads * dh], exp[:, : heads * dh]) <= TOL_F32


@pytest.mark.parametrize("dt", ["fp32", "bf16-stream", "bf16-wide"])
def test_config3_shape_subset(gpu, oracle, dt, monkeypatch):
    """Config 3's attention shape (1024 tokens, 12x64, rope_partial_factor 0.5, gate on, every row
    known = bidirectional, left padding U{0..256}) on 2 series."""
    if "-" in dt:
        monkeypatch.setenv("JITCAST_HIP_LP_KERNEL", dt.split("-")[1])
    dt = dt.split("-")[0]
    rows, enc, heads, dh, d, rope_dim = 2, 1024, 12, 64, 768, 32
    qkv = cases.qkv(101, rows * enc, d, std=0.6)
    kv, known, position = cases.ts_layout(101, rows, enc, enc, 0, 1.0, max_start=256)
    g = cases.qkv(102, rows * enc, d)[:, :d].copy()
    got = _run(qkv, kv, known, position, g, rows, enc, enc, enc, heads, dh, d, rope_dim, DTYPES[dt])
    exp = _expected(oracle, qkv, kv, known, position, g, rows, enc, enc, enc, heads, dh, d, rope_dim)
    err = oracle.rel_max_error(got, exp)
    print(f"config-3 subset {dt} rel err {err:.3e}", flush=True)
    assert err <= (TOL_F32 if dt == "fp32" else TOL_LP)


@pytest.mark.parametrize("dt", ["fp32", "bf16", "fp16"])
def test_standalone_gate(gpu, oracle, dt):
    att = cases.qkv(103, 333, 3)[:, :7].copy()
    g = cases.qkv(104, 333, 3)[:, :7].copy() * 3
    a = torch.from_numpy(att).cuda().to(DTYPES[dt])
    timestral.gate(a, torch.from_numpy(g).cuda().to(DTYPES[dt]))
    torch.cuda.synchronize()
    rounded = [torch.from_numpy(x).to(DTYPES[dt]).float().numpy() for x in (att, g)]
    exp = oracle.ts_gate(*rounded)
    tol = 1e-6 if dt == "fp32" else 1e-2
    assert oracle.rel_max_error(a.float().cpu().numpy(), exp) <= tol


def test_rejects_bad_arguments(gpu):
    dev = torch.device("cuda:0")
    q = torch.zeros(8 * 3 * 64, device=dev)
    o = torch.zeros(8 * 64, device=dev)
    kv = torch.ones(8, dtype=torch.int32, device=dev)
    with pytest.raises(JitcastArgumentError, match="token counts"):
        timestral.time_attention(q, o, kv, None, None, None, None, 1, 8, 9, 8, 1, 64, 64)
    with pytest.raises(JitcastArgumentError, match="head width"):
        timestral.time_attention(q, o, kv, None, None, None, None, 1, 8, 8, 8, 1, 60, 64)
    with pytest.raises(JitcastArgumentError, match="head width"):
        timestral.time_attention(q.bfloat16(), o.bfloat16(), kv, None, None, None, None, 1, 8, 8, 8, 1, 24, 64)
