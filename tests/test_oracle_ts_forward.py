"""Pins of the oracle's Timestral block forward (CpuTimestral.predictBlock from the patch tokens to the
head's raw outputs, J/timestral/cpu/CpuTimestral.java:127-188) and of its new pieces (Ops.silu, the
SwiGLU activation, the SiLU residual block) against closed forms and a float64 restatement built on
tests/brute.py's attention. CPU only."""
import numpy as np
import pytest

from jitcast_amd import timestral_model as tm
from tests import brute, cases

pytestmark = pytest.mark.usefixtures("oracle")

TINY = tm.TimestralConfig(patch_size=8, d_model=32, num_heads=2, mlp_hidden_dim=48,
                          layers=((True, False), (False, True)), quantiles=(0.1, 0.5, 0.9))


def test_silu_closed_forms(oracle):
    x = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 1e-8], np.float32)
    got = oracle.silu(x)
    exp = np.array([0.0, 1.0 / (1.0 + np.exp(-1.0)), -1.0 / (1.0 + np.exp(1.0)), 30.0, -30.0 * np.exp(-30.0) / (1 + np.exp(-30.0)),
                    5e-9], np.float64)
    np.testing.assert_allclose(got, exp.astype(np.float32), rtol=2e-7, atol=0)
    assert got[0] == 0 and got[3] == np.float32(30.0)


def test_swiglu_gate_half_first(oracle):
    """act = silu(first half) * second half: a unit second half returns silu of the first, a zero
    first half returns 0 whatever the second."""
    r = np.random.default_rng(0)
    a = r.standard_normal((5, 7)).astype(np.float32)
    up = np.concatenate([a, np.ones((5, 7), np.float32)], axis=1)
    np.testing.assert_array_equal(oracle.swiglu(up, 7), oracle.silu(a))
    up = np.concatenate([np.zeros((5, 7), np.float32), a], axis=1)
    np.testing.assert_array_equal(oracle.swiglu(up, 7), np.zeros((5, 7), np.float32))


def _lin(x, w, b=None):
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    return y if b is None else y + np.asarray(b, np.float64)


def _rms(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps) * np.asarray(w, np.float64)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _res(x, w, pre):
    hid = _silu(_lin(x, w[pre + "_hidden_w"], w.get(pre + "_hidden_b")))
    return _lin(hid, w[pre + "_output_w"], w.get(pre + "_output_b")) + _lin(x, w[pre + "_residual_w"],
                                                                          w.get(pre + "_residual_b"))


def _brute_forward(tokens, w, c, kv, known, position, group, role, covariates, rows, enc, h):
    n, d, heads, dh = enc + h, c.d_model, c.num_heads, c.head_dim
    ll = enc - h if covariates else enc
    emb = _res(tokens, w, "embed")
    x = np.zeros((rows * n, d))
    for i in range(rows):
        x[i * n: i * n + enc] = emb[i * enc: (i + 1) * enc]
        x[i * n + enc: (i + 1) * n] = w["query"]
    for lw in w["layers"]:
        for a in lw["attentions"]:
            hn = _rms(x, a["norm"], c.norm_eps)
            qkv = _lin(hn, a["qkv"]).astype(np.float32)
            if a["time"]:
                att = brute.ts_time(qkv, kv, known, position, rows, enc, ll, n, heads, dh, d, c.rope_dim, c.rope_theta)
            else:
                att = brute.ts_variate(qkv, kv, group, role, covariates, rows, enc, n, heads, dh, d)
            att = att.astype(np.float64)
            if a["gate"] is not None:
                att = att / (1.0 + np.exp(-_lin(hn, a["gate"])))
            x = x + _lin(att, a["wo"])
        hn = _rms(x, lw["mlp_norm"], c.norm_eps)
        f = lw["down"].shape[1]
        up = _lin(hn, lw["up"])
        x = x + _lin(_silu(up[:, :f]) * up[:, f:], lw["down"])
    y = _rms(x, w["out_norm"], c.norm_eps)
    dec = np.concatenate([y[i * n + enc: (i + 1) * n] for i in range(rows)])
    return _res(dec, w, "head")


@pytest.mark.parametrize("covariates", [False, True])
def test_forward_matches_brute_force(oracle, covariates):
    c = TINY
    rows, enc, h = 6, 5, 2
    ll = enc - h if covariates else enc
    kv, known, position = cases.ts_layout(3, rows, enc, ll, h, known_frac=0.4 if covariates else 0.0)
    group = np.array([0, 0, 0, 1, 1, 1], np.int32)
    role = np.array([0, 1, 2, 0, 1, 1] if covariates else [0] * rows, np.int32)
    w = tm.random_weights(c, seed=1, std=0.2)
    r = np.random.default_rng(2)
    tok = r.standard_normal((rows * enc, 2 * c.patch_size)).astype(np.float32)
    got = oracle.ts_forward_raw(tok, w, kv, known, position, group, role, covariates, rows, enc, ll, h, c.num_heads,
                                c.head_dim, c.rope_dim, c.norm_eps, c.rope_theta)
    exp = _brute_forward(tok, w, c, kv, known, position, group, role, covariates, rows, enc, h)
    assert got.shape == (rows * h, c.patch_size * c.num_quantiles)
    err = np.max(np.abs(got - exp)) / np.max(np.abs(exp))
    assert err < 2e-5, err
