"""jc_ts_block_layout (the host BlockLayout.of) against an independent pure-Python restatement of
BlockLayout.java:77-148 and 203-207, on seeded blocks with and without covariates (CPU only)."""
import numpy as np
import pytest

from jitcast_amd import JitcastArgumentError, rng, timestral
from tests import cases


def _reference_layout(observed, future, group, role, h, patch, cov_enabled, attend_missing):
    rows, t = observed.shape
    cov = role is not None and cov_enabled and any(x != 0 for x in role)
    ll = t // patch
    if cov:
        fut = future if future is not None else np.zeros((rows, h * patch), bool)
        window = np.concatenate([observed.astype(bool), fut.astype(bool)], axis=1)
    else:
        window = observed.astype(bool)
    enc = window.shape[1] // patch
    valid = np.zeros((rows, enc), bool)
    first = []
    for i in range(rows):
        started = False
        f = enc
        for p in range(enc):
            anyobs = bool(window[i, p * patch:(p + 1) * patch].any())
            if anyobs and f == enc:
                f = p
            started = started or anyobs
            valid[i, p] = started if attend_missing else anyobs
        first.append(f)
    gfirst = {}
    for i in range(rows):
        gfirst[group[i]] = min(gfirst.get(group[i], enc), first[i])
    pos = np.zeros((rows, enc + h), np.int64)
    for i in range(rows):
        f = gfirst[group[i]]
        f = 0 if f == enc else f
        for k in range(enc + h):
            pos[i, k] = (k if k < enc else ll + k - enc) - f + enc
    known = np.array([1 if cov and role[i] == 2 else 0 for i in range(rows)])
    return enc, cov, valid.astype(np.int32), known, pos


@pytest.mark.parametrize("cov_enabled,with_role,with_future,attend", [
    (True, True, True, True), (True, True, False, True), (True, False, False, True), (False, True, True, True),
    (True, True, True, False),
])
def test_block_layout_matches_restatement(cov_enabled, with_role, with_future, attend):
    rows, patch, ll, h = 9, 4, 7, 3
    t = ll * patch
    obs = rng.uniform(rng.stream_seed(5, 7), rows * t).reshape(rows, t) < 0.5
    obs[0, :] = False  # a row that never observes
    obs[1, : 3 * patch] = False  # a late start
    group = cases.group_sizes(5, rows, 2, 4)
    role = np.floor(rng.uniform(rng.stream_seed(5, 8), rows) * 3).astype(np.int32) if with_role else None
    fut = (rng.uniform(rng.stream_seed(5, 9), rows * h * patch).reshape(rows, h * patch) < 0.7) if with_future else None
    got = timestral.block_layout(obs, group, h, patch, role, fut, cov_enabled, attend)
    exp = _reference_layout(obs, fut, group, role, h, patch, cov_enabled, attend)
    assert got[0] == exp[0] and got[1] == exp[1]
    for a, b in zip(got[2:], exp[2:]):
        np.testing.assert_array_equal(a, b)


def test_block_layout_errors_mirror_block_layout_of():
    obs = np.ones((2, 10), bool)
    with pytest.raises(JitcastArgumentError, match="not a multiple of the patch size"):
        timestral.block_layout(obs, [0, 0], 1, 4)
    with pytest.raises(JitcastArgumentError, match="horizon patches must be >= 1"):
        timestral.block_layout(np.ones((2, 8), bool), [0, 0], 0, 4)
    with pytest.raises(JitcastArgumentError, match="decodes at most"):
        timestral.block_layout(np.ones((2, 8), bool), [0, 0], 5, 4, role=[0, 2], block_size=4)
