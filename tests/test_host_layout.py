"""Host-side layout helpers of libjitcast_hip (CPU only): the live mask, the group order and the
group bounds, against the oracle and the rules of ModelLayout.java:104-114 and
Chronos2Forward.java:178-194, 475-489."""
import numpy as np
import pytest

from jitcast_amd import JitcastArgumentError, chronos2
from tests import cases


def test_live_mask_matches_oracle(oracle):
    rows, nc, patch, h = 5, 7, 4, 3
    w = np.arange(rows * nc * patch, dtype=np.float32).reshape(rows, nc * patch)
    rnd = cases.random_live(3, rows, nc * patch, 0.3)
    w[rnd == 1] = np.nan
    w[2, :] = np.nan
    for reg in (0, 1):
        np.testing.assert_array_equal(chronos2.live_mask(w, nc, patch, reg, h), oracle.c2_live(w, rows, nc, patch, reg, h))


def test_group_order_first_appearance():
    g = np.array([4, 2, 4, 9, 2, 9, 9], np.int32)
    order = chronos2.group_order(g)
    np.testing.assert_array_equal(order, [0, 2, 1, 4, 3, 5, 6])
    assert chronos2.group_order(np.array([1, 1, 0, 0, 5], np.int32)) is None


def test_group_bounds():
    s, e = chronos2.group_bounds(np.array([3, 3, 1, 7, 7, 7], np.int32))
    np.testing.assert_array_equal(s, [0, 0, 2, 3, 3, 3])
    np.testing.assert_array_equal(e, [2, 2, 3, 6, 6, 6])
    with pytest.raises(JitcastArgumentError, match="not contiguous"):
        chronos2.group_bounds(np.array([1, 2, 1], np.int32))


def test_order_then_bounds_gives_contiguous_groups():
    g = cases.group_sizes(5, 40, 1, 6)
    perm = np.random.default_rng(0).permutation(40)
    shuffled = g[perm]
    order = chronos2.group_order(shuffled)
    s, e = chronos2.group_bounds(shuffled[order])
    for i in range(40):
        assert np.all(shuffled[order][s[i]:e[i]] == shuffled[order][i])
