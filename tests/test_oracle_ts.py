"""Pins the C oracle's Timestral stages (CPU only).

The numpy float64 brute force (tests/brute.py) restates BlockLayout.timeAllowed / variateAllowed and
CpuTimestral's attention independently of the oracle's code; torch's SDPA pins the reduction where
the mask degenerates to plain attention; the invariants pin causality, known rows, the decoder's
context limit and the partial RoPE; the table is checked against a float64 recomputation of the
reference's float rounding (CpuTimestral.java:107-116, TimestralForward.java:599-610).
"""
import numpy as np
import pytest
import torch

from jitcast_amd import timestral
from tests import brute, cases


@pytest.mark.parametrize("dh,rope_dim", [(64, 32), (64, 64), (32, 16), (128, 64), (24, 12)])
def test_inv_freq_partial_bit_exact(oracle, dh, rope_dim):
    got = oracle.ts_inv_freq(dh, rope_dim)
    np.testing.assert_array_equal(got, brute.inv_freq(dh, rope_dim=rope_dim))
    assert not np.any(got[rope_dim // 2:])  # dims past rope_dim/2 never rotate


def test_rope_table_rows_are_positions(oracle):
    enc, h, dh, rope_dim = 40, 3, 64, 32
    n = enc + h
    t = timestral.rope_table(enc, n, dh, rope_dim)
    assert t.shape == (enc + n, dh)
    inv = oracle.ts_inv_freq(dh, rope_dim)
    pos = (np.arange(enc + n) - enc).astype(np.float32)
    ang = (pos[:, None] * inv[None, :]).astype(np.float64)  # float product, then double cos/sin
    np.testing.assert_array_equal(t[:, : dh // 2], np.cos(ang).astype(np.float32))
    np.testing.assert_array_equal(t[:, dh // 2:], np.sin(ang).astype(np.float32))
    # position 0 (row enc) is the identity; the unrotated dims are the identity at every position
    np.testing.assert_array_equal(t[enc], np.r_[np.ones(dh // 2), np.zeros(dh // 2)].astype(np.float32))
    np.testing.assert_array_equal(t[:, rope_dim // 2: dh // 2], 1.0)
    np.testing.assert_array_equal(t[:, dh // 2 + rope_dim // 2:], 0.0)


TIME_CASES = [
    # rows, enc, ll, h, heads, dh, d, rope_dim, known_frac
    (3, 20, 20, 4, 2, 32, 64, 16, 0.0),
    (4, 24, 20, 2, 2, 16, 40, 8, 0.5),  # covariates: ll < enc, some known rows
    (2, 33, 33, 0, 3, 32, 96, 32, 0.0),  # encoder only, causal
    (2, 17, 17, 5, 1, 64, 64, 32, 1.0),  # every row known (bidirectional encoder)
]


@pytest.mark.parametrize("rows,enc,ll,h,heads,dh,d,rope_dim,known_frac", TIME_CASES)
def test_time_attention_matches_brute_force(oracle, rows, enc, ll, h, heads, dh, d, rope_dim, known_frac):
    n = enc + h
    qkv = cases.qkv(61, rows * n, d)
    kv, known, pos = cases.ts_layout(61, rows, enc, ll, h, known_frac)
    got = oracle.ts_time_attention(qkv, kv, known, pos, rows, enc, ll, n, heads, dh, d, rope_dim)
    exp = brute.ts_time(qkv, kv, known, pos, rows, enc, ll, n, heads, dh, d, rope_dim)
    assert oracle.rel_max_error(got, exp) < 1e-6


def test_time_attention_equals_sdpa_when_bidirectional(oracle):
    """Known rows with every key valid and no decoder tokens: plain attention scaled by 1/sqrt(dh)."""
    rows, enc, heads, dh, d, rope_dim = 2, 30, 2, 32, 64, 16
    qkv = cases.qkv(67, rows * enc, d)
    kv = np.ones((rows, enc), np.int32)
    known = np.ones(rows, np.int32)
    pos = np.broadcast_to(np.arange(enc, dtype=np.int32) - 3, (rows, enc)).copy()
    got = oracle.ts_time_attention(qkv, kv, known, pos, rows, enc, enc, enc, heads, dh, d, rope_dim)
    q, k, v = brute.split_qkv(qkv, rows, enc, heads, dh, d)
    inv = brute.inv_freq(dh, rope_dim=rope_dim)
    qr = torch.from_numpy(brute.rope_float(q, pos, inv).astype(np.float64)).permute(0, 2, 1, 3)
    kr = torch.from_numpy(brute.rope_float(k, pos, inv).astype(np.float64)).permute(0, 2, 1, 3)
    vv = torch.from_numpy(v.astype(np.float64)).permute(0, 2, 1, 3)
    ref = torch.nn.functional.scaled_dot_product_attention(qr, kr, vv, scale=1.0 / np.sqrt(dh))
    ref = ref.permute(0, 2, 1, 3).reshape(rows * enc, heads * dh).numpy()
    assert oracle.rel_max_error(got, ref) < 1e-6


def test_time_attention_causal_and_known_invariants(oracle):
    rows, enc, ll, h, heads, dh, d, rope_dim = 2, 24, 24, 4, 2, 32, 64, 16
    n = enc + h
    qkv = cases.qkv(71, rows * n, d)
    kv = np.ones((rows, enc), np.int32)
    known = np.array([0, 1], np.int32)
    pos = cases.ts_layout(71, rows, enc, ll, h, 0.0, max_start=0)[2]
    base = oracle.ts_time_attention(qkv, kv, known, pos, rows, enc, ll, n, heads, dh, d, rope_dim)
    base = base.reshape(rows, n, d)
    # perturb the k and v of encoder tokens 12.. : row 0 (causal) keeps outputs 0..11 bit for bit,
    # row 1 (known, bidirectional) changes there
    p = qkv.copy().reshape(rows, n, 3 * d)
    p[:, 12:enc, d:] += 1.0
    pert = oracle.ts_time_attention(p.reshape(rows * n, -1), kv, known, pos, rows, enc, ll, n, heads, dh, d,
                                    rope_dim).reshape(rows, n, d)
    np.testing.assert_array_equal(pert[0, :12], base[0, :12])
    assert np.abs(pert[1, :12] - base[1, :12]).max() > 1e-3
    # decoder queries never read encoder keys >= ll: with ll = 20, perturbing keys 20..enc-1 leaves
    # every decoder output of row 0 unchanged
    ll2 = 20
    b2 = oracle.ts_time_attention(qkv, kv, known, pos, rows, enc, ll2, n, heads, dh, d, rope_dim).reshape(rows, n, d)
    p2 = qkv.copy().reshape(rows, n, 3 * d)
    p2[:, ll2:enc, d:] += 1.0
    o2 = oracle.ts_time_attention(p2.reshape(rows * n, -1), kv, known, pos, rows, enc, ll2, n, heads, dh, d,
                                  rope_dim).reshape(rows, n, d)
    np.testing.assert_array_equal(o2[:, enc:], b2[:, enc:])
    # an encoder query whose own patch is not a valid key, with no valid key before it, reads itself
    kv3 = kv.copy()
    kv3[0, :5] = 0
    o3 = oracle.ts_time_attention(qkv, kv3, known, pos, rows, enc, ll, n, heads, dh, d, rope_dim).reshape(rows, n, d)
    v = qkv.reshape(rows, n, 3 * d)[:, :, 2 * d:]
    np.testing.assert_array_equal(o3[0, :5, : heads * dh], v[0, :5, : heads * dh])


def test_gate_matches_float64_sigmoid(oracle):
    att = cases.qkv(73, 50, 4)[:, :8].copy()
    g = cases.qkv(74, 50, 4)[:, :8] * 4
    got = oracle.ts_gate(att, g)
    exp = (att.astype(np.float64) * (1.0 / (1.0 + np.exp(-g.astype(np.float64))))).astype(np.float32)
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=0)


VARIATE_CASES = [
    # rows, enc, h, heads, dh, d, group sizes lo..hi, covariates
    (12, 6, 2, 2, 32, 64, 1, 5, 0),
    (15, 5, 3, 2, 16, 40, 2, 6, 1),
]


@pytest.mark.parametrize("rows,enc,h,heads,dh,d,lo,hi,cov", VARIATE_CASES)
def test_variate_attention_matches_brute_force(oracle, rows, enc, h, heads, dh, d, lo, hi, cov):
    n = enc + h
    qkv = cases.qkv(79, rows * n, d)
    kv = cases.random_live(79, rows, enc, 0.7)
    group = cases.group_sizes(79, rows, lo, hi)
    # roles cycle TARGET(0), PAST(1), KNOWN(2) (BlockInput.java:35-37)
    role = (np.arange(rows) % 3).astype(np.int32) if cov else np.zeros(rows, np.int32)
    got = oracle.ts_variate_attention(qkv, kv, group, role, cov, rows, enc, n, heads, dh, d)
    exp = brute.ts_variate(qkv, kv, group, role, cov, rows, enc, n, heads, dh, d)
    assert oracle.rel_max_error(got, exp) < 1e-6
