"""Pins the C oracle's Chronos-2 stages (CPU only).

Each check is chosen so that a plausible mistake fails it: the numpy float64 brute force (shares
no code with the oracle) catches index, sign and transposition errors; torch's SDPA pins the
attention reduction itself; the invariants pin masking and the no-key case; the table checks pin
the RoPE rounding of CpuChronos2.java:102-111 / Chronos2Forward.java:467-474.
"""
import numpy as np
import pytest
import torch

from tests import brute, cases


def test_inv_freq_bit_exact(oracle):
    for dh in (16, 32, 48, 64, 128):
        np.testing.assert_array_equal(oracle.c2_inv_freq(dh), brute.inv_freq(dh))


def test_rope_table_rounding(oracle):
    n, dh = 600, 64
    t = oracle.c2_rope_table(n, dh)
    inv = brute.inv_freq(dh)
    ang = (np.arange(n, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)
    np.testing.assert_array_equal(t[:, :32], np.cos(ang).astype(np.float32))
    np.testing.assert_array_equal(t[:, 32:], np.sin(ang).astype(np.float32))
    # position 0 is the identity rotation
    np.testing.assert_array_equal(t[0], np.r_[np.ones(32), np.zeros(32)].astype(np.float32))
    # every (cos, sin) pair is a rotation: cos^2 + sin^2 = 1 to float precision
    np.testing.assert_allclose(t[:, :32].astype(np.float64) ** 2 + t[:, 32:].astype(np.float64) ** 2, 1.0,
                               atol=4e-7)


def test_rope_relative_position(oracle):
    """<R_m q, R_n k> depends only on m - n (to float precision of the rounded table)."""
    dh = 64
    t = oracle.c2_rope_table(200, dh).astype(np.float64)
    rq = np.random.default_rng(3).standard_normal(dh)
    rk = np.random.default_rng(4).standard_normal(dh)

    def rot(x, p):
        c, s = t[p, :32], t[p, 32:]
        return np.r_[x[:32] * c - x[32:] * s, x[32:] * c + x[:32] * s]

    base = rot(rq, 7) @ rot(rk, 3)
    for shift in (1, 20, 150):
        assert abs(rot(rq, 7 + shift) @ rot(rk, 3 + shift) - base) < 5e-5 * (1 + abs(base))
    # norm preserved
    assert abs(np.linalg.norm(rot(rq, 123)) - np.linalg.norm(rq)) < 1e-6 * np.linalg.norm(rq)


CASES = [
    # rows, n, heads, dh, inner, live kind
    (2, 37, 2, 64, 128, "pad"),
    (3, 33, 3, 32, 100, "pad"),
    (2, 20, 2, 48, 96, "random"),
    (1, 5, 1, 16, 16, "all"),
    (2, 64, 2, 64, 128, "random"),
]


def _live(kind, seed, rows, n):
    if kind == "pad":
        return cases.left_pad_live(seed, rows, n, n // 2)
    if kind == "random":
        return cases.random_live(seed, rows, n, 0.6)
    return np.ones((rows, n), np.int32)


@pytest.mark.parametrize("rows,n,heads,dh,inner,kind", CASES)
def test_time_attention_matches_brute_force(oracle, rows, n, heads, dh, inner, kind):
    qkv = cases.qkv(11, rows * n, inner)
    live = _live(kind, 11, rows, n)
    got = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner)
    exp = brute.c2_time(qkv, live, rows, n, heads, dh, inner)
    assert oracle.rel_max_error(got, exp) < 1e-6


def test_time_attention_equals_sdpa_when_all_live(oracle):
    rows, n, heads, dh, inner = 2, 40, 3, 64, 192
    qkv = cases.qkv(5, rows * n, inner)
    live = np.ones((rows, n), np.int32)
    got = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner)
    q, k, v = brute.split_qkv(qkv, rows, n, heads, dh, inner)
    pos = np.broadcast_to(np.arange(n), (rows, n))
    inv = brute.inv_freq(dh)
    qr = torch.from_numpy(brute.rope_float(q, pos, inv).astype(np.float64)).permute(0, 2, 1, 3)
    kr = torch.from_numpy(brute.rope_float(k, pos, inv).astype(np.float64)).permute(0, 2, 1, 3)
    vv = torch.from_numpy(v.astype(np.float64)).permute(0, 2, 1, 3)
    ref = torch.nn.functional.scaled_dot_product_attention(qr, kr, vv, scale=1.0)
    ref = ref.permute(0, 2, 1, 3).reshape(rows * n, heads * dh).numpy()
    assert oracle.rel_max_error(got, ref) < 1e-6


def test_time_attention_invariants(oracle):
    rows, n, heads, dh, inner = 2, 24, 2, 64, 128
    qkv = cases.qkv(7, rows * n, inner)
    # exactly one live key: every query outputs that key's v, bit for bit
    live = np.zeros((rows, n), np.int32)
    live[0, 5] = 1
    live[1, 23] = 1
    out = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner).reshape(rows, n, inner)
    v = qkv.reshape(rows, n, 3 * inner)[:, :, 2 * inner:]
    np.testing.assert_array_equal(out[0], np.broadcast_to(v[0, 5], (n, inner)))
    np.testing.assert_array_equal(out[1], np.broadcast_to(v[1, 23], (n, inner)))
    # q = 0: the mean of the live v
    z = qkv.copy().reshape(rows, n, 3 * inner)
    z[:, :, :inner] = 0
    live = cases.random_live(9, rows, n, 0.5)
    live[:, -1] = 1
    out = oracle.c2_time_attention(z.reshape(rows * n, -1), live, rows, n, heads, dh, inner).reshape(rows, n, inner)
    for r in range(rows):
        mean = z[r, live[r] == 1, 2 * inner:].astype(np.float64).mean(axis=0)
        np.testing.assert_allclose(out[r], np.broadcast_to(mean, (n, inner)), rtol=0, atol=1e-6)
    # perturbing k and v at dead keys changes nothing
    base = oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner)
    p = qkv.copy().reshape(rows, n, 3 * inner)
    p[live == 0, inner:] += 100.0
    again = oracle.c2_time_attention(p.reshape(rows * n, -1), live, rows, n, heads, dh, inner)
    np.testing.assert_array_equal(base, again)
    # no live key: zeros
    none = oracle.c2_time_attention(qkv, np.zeros((rows, n), np.int32), rows, n, heads, dh, inner)
    assert not np.any(none)


GROUP_CASES = [
    (12, 5, 2, 64, 128, 1, 4),
    (30, 3, 3, 32, 96, 1, 9),
    (9, 4, 1, 16, 16, 9, 9),
]


@pytest.mark.parametrize("rows,n,heads,dh,inner,lo,hi", GROUP_CASES)
def test_group_attention_matches_brute_force(oracle, rows, n, heads, dh, inner, lo, hi):
    qkv = cases.qkv(13, rows * n, inner)
    live = cases.random_live(13, rows, n, 0.7)
    group = cases.group_sizes(13, rows, lo, hi)
    got = oracle.c2_group_attention(qkv, live, group, rows, n, heads, dh, inner)
    exp = brute.c2_group(qkv, live, group, rows, n, heads, dh, inner)
    assert oracle.rel_max_error(got, exp) < 1e-6


def test_group_attention_non_contiguous_ids_match_brute_force(oracle):
    rows, n, heads, dh, inner = 10, 3, 2, 32, 64
    qkv = cases.qkv(17, rows * n, inner)
    live = cases.random_live(17, rows, n, 0.8)
    group = np.array([3, 1, 3, 2, 1, 3, 2, 2, 1, 7], np.int32)
    got = oracle.c2_group_attention(qkv, live, group, rows, n, heads, dh, inner)
    exp = brute.c2_group(qkv, live, group, rows, n, heads, dh, inner)
    assert oracle.rel_max_error(got, exp) < 1e-6


def test_group_attention_invariants(oracle):
    rows, n, heads, dh, inner = 8, 4, 2, 64, 128
    qkv = cases.qkv(19, rows * n, inner)
    live = np.ones((rows, n), np.int32)
    group = np.array([0, 1, 1, 1, 2, 2, 3, 3], np.int32)
    out = oracle.c2_group_attention(qkv, live, group, rows, n, heads, dh, inner).reshape(rows, n, inner)
    v = qkv.reshape(rows, n, 3 * inner)[:, :, 2 * inner:]
    # a group of one row reads only itself
    np.testing.assert_array_equal(out[0], v[0])
    # a slot nobody in the group observes gets zeros
    dead = live.copy()
    dead[4:6, 2] = 0
    o2 = oracle.c2_group_attention(qkv, dead, group, rows, n, heads, dh, inner).reshape(rows, n, inner)
    assert not np.any(o2[4:6, 2])
    # groups are independent: perturbing group 2 leaves the others bit-identical
    p = qkv.copy().reshape(rows, n, 3 * inner)
    p[4:6] += 3.0
    o3 = oracle.c2_group_attention(p.reshape(rows * n, -1), live, group, rows, n, heads, dh, inner).reshape(
        rows, n, inner)
    np.testing.assert_array_equal(np.delete(o3, [4, 5], axis=0), np.delete(out, [4, 5], axis=0))
    # equivariant under a permutation of rows (with their ids)
    perm = np.array([3, 0, 7, 1, 5, 2, 6, 4])
    q = qkv.reshape(rows, n, 3 * inner)[perm].reshape(rows * n, -1)
    o4 = oracle.c2_group_attention(q, live[perm], group[perm], rows, n, heads, dh, inner).reshape(rows, n, inner)
    np.testing.assert_allclose(o4, out[perm], rtol=0, atol=2e-6)


def test_live_mask_follows_model_layout(oracle):
    """ModelLayout.java:104-114: a context patch is live if any step is observed; REG/future always."""
    rows, nc, patch, h = 2, 4, 3, 2
    w = np.ones((rows, nc * patch), np.float32)
    w[0, 0:3] = np.nan  # patch 0 of row 0 unobserved
    w[1, 3:5] = np.nan  # patch 1 of row 1 partly observed -> still live
    w[1, 9:12] = np.nan  # patch 3 of row 1 unobserved
    live = oracle.c2_live(w, rows, nc, patch, 1, h)
    np.testing.assert_array_equal(live, [[0, 1, 1, 1, 1, 1, 1], [1, 1, 1, 0, 1, 1, 1]])
