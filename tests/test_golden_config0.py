"""Config 0's committed fixture (tests/golden/config0.npz, written by tests/golden/make_config0.py):
the generator still draws the stored inputs, and the oracle (Chronos2Pipeline over CpuChronos2.forward)
still produces the stored quantiles and per-layer activations. The GPU engine is held to the same
fixture in tests/test_gpu_engine.py."""
from pathlib import Path

import numpy as np

from jitcast_amd import synthetic

FIXTURE = Path(__file__).resolve().parent / "golden" / "config0.npz"


def test_fixture_inputs_are_the_generators():
    g = np.load(FIXTURE)
    np.testing.assert_array_equal(g["inputs"], synthetic.c2_config0_series())
    x = g["inputs"].astype(np.float64)
    # sines of amplitude <= 2 each, a trend under 0.01 * 511, noise N(0, 0.1)
    assert np.abs(x).max() < 2 * 2 + 0.01 * 511 + 1.0
    assert g["quantiles"].shape == (4, 21, 64) and g["layers"].shape == (6, 4 * 37, 512)


def test_oracle_reproduces_the_fixture(oracle):
    import tests.golden.make_config0 as mk

    g = np.load(FIXTURE)
    w = synthetic.c2_portable_weights(mk.CONFIG0, seed=0)
    q, layers = mk.run(w, g["inputs"])
    assert oracle.rel_max_error(q, g["quantiles"]) <= 1e-6
    assert oracle.rel_max_error(layers, g["layers"]) <= 1e-6
    # non-crossing is not a property of an untrained model's raw quantiles; finiteness is
    assert np.isfinite(q).all()
