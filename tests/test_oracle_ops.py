"""Pins of the oracle's layer ops (Ops.Linear.apply, Ops.rmsNorm, Ops.reluInPlace, Ops.addInPlace;
J/cpu/Ops.java:33-88) and of its encoder-layer composition (CpuChronos2.forward,
J/chronos2/cpu/CpuChronos2.java:150-161) against independent float64 numpy restatements.
"""
import numpy as np
import pytest

from tests import brute, cases

pytestmark = pytest.mark.usefixtures("oracle")


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("rows,inn,out", [(1, 16, 3), (17, 40, 9), (33, 7, 65)])
@pytest.mark.parametrize("bias", [False, True])
def test_linear_is_x_times_w_transposed(oracle, rows, inn, out, bias):
    r = _rng(rows * 100 + inn)
    x = r.standard_normal((rows, inn)).astype(np.float32)
    w = r.standard_normal((out, inn)).astype(np.float32)  # PyTorch [out, in]: a transposed use fails here
    b = r.standard_normal(out).astype(np.float32) if bias else None
    exp = x.astype(np.float64) @ w.astype(np.float64).T + (0 if b is None else b.astype(np.float64))
    got = oracle.linear(x, w, b)
    assert got.shape == (rows, out)
    np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-6)


def test_linear_threads_do_not_change_results(oracle):
    r = _rng(5)
    x = r.standard_normal((70, 32)).astype(np.float32)
    w = r.standard_normal((24, 32)).astype(np.float32)
    np.testing.assert_array_equal(oracle.linear(x, w, threads=1), oracle.linear(x, w, threads=4))


@pytest.mark.parametrize("with_w", [False, True])
def test_rms_norm_closed_form(oracle, with_w):
    r = _rng(7)
    x = (r.standard_normal((9, 24)) * 3).astype(np.float32)
    w = r.standard_normal(24).astype(np.float32) if with_w else None
    eps = 1e-6
    x64 = x.astype(np.float64)
    inv = (1.0 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps)).astype(np.float32)
    exp = x * inv * (w if with_w else np.float32(1))
    np.testing.assert_allclose(oracle.rms_norm(x, w, eps), exp, rtol=1e-6, atol=0)
    # invariants: rows come out with mean square ~ 1 (w = None), and scaling a row does not change it
    if not with_w:
        y = oracle.rms_norm(x, None, 0.0)
        np.testing.assert_allclose((y.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-5)
        np.testing.assert_allclose(oracle.rms_norm(4 * x, None, 0.0), y, rtol=1e-6)


def test_relu_and_add(oracle):
    x = np.array([-2.0, -0.0, 0.0, 1.5, np.nan, np.inf, -np.inf], np.float32)
    y = oracle.relu(x)
    assert np.isnan(y[4])
    np.testing.assert_array_equal(y[[0, 1, 2, 3, 5, 6]], np.array([0, 0, 0, 1.5, np.inf, 0], np.float32))
    a = np.arange(5, dtype=np.float32)
    np.testing.assert_array_equal(oracle.add(a, 2 * a), 3 * a)


def _layer_weights(seed, d, inner, dff, bias=False):
    r = _rng(seed)

    def m(o, i):
        return (r.standard_normal((o, i)) * (1.0 / np.sqrt(i))).astype(np.float32)

    w = {
        "time_norm": (1 + 0.1 * r.standard_normal(d)).astype(np.float32),
        "time_qkv": m(3 * inner, d), "time_o": m(d, inner),
        "group_norm": (1 + 0.1 * r.standard_normal(d)).astype(np.float32),
        "group_qkv": m(3 * inner, d), "group_o": m(d, inner),
        "mlp_norm": (1 + 0.1 * r.standard_normal(d)).astype(np.float32),
        "wi": m(dff, d), "wo": m(d, dff),
    }
    if bias:
        for k, o in (("time_qkv_bias", 3 * inner), ("time_o_bias", d), ("group_qkv_bias", 3 * inner),
                     ("group_o_bias", d), ("wi_bias", dff), ("wo_bias", d)):
            w[k] = (0.1 * r.standard_normal(o)).astype(np.float32)
    return w


def _brute_layer(x, w, live, group, rows, n, heads, dh, eps):
    """float64 restatement of the layer: rmsNorm, linears, brute attention, ReLU, residual adds."""
    inner = heads * dh

    def rms(v, g):
        return v / np.sqrt((v * v).mean(axis=1, keepdims=True) + eps) * g.astype(np.float64)

    def lin(v, name):
        y = v @ w[name].astype(np.float64).T
        b = w.get(name + "_bias")
        return y if b is None else y + b.astype(np.float64)

    x = x.astype(np.float64)
    qkv = lin(rms(x, w["time_norm"]), "time_qkv").astype(np.float32)
    x = x + lin(brute.c2_time(qkv, live, rows, n, heads, dh, inner), "time_o")
    qkv = lin(rms(x, w["group_norm"]), "group_qkv").astype(np.float32)
    x = x + lin(brute.c2_group(qkv, live, group, rows, n, heads, dh, inner), "group_o")
    act = np.maximum(lin(rms(x, w["mlp_norm"]), "wi"), 0.0)
    return x + lin(act, "wo")


@pytest.mark.parametrize("bias", [False, True])
def test_layer_composition_matches_brute_force(oracle, bias):
    rows, n, heads, dh, d, dff = 5, 11, 2, 8, 16, 32
    inner = heads * dh
    w = _layer_weights(11, d, inner, dff, bias)
    x = _rng(12).standard_normal((rows * n, d)).astype(np.float32)
    live = cases.left_pad_live(12, rows, n, 4)
    group = np.array([0, 0, 1, 1, 1], np.int32)
    got = oracle.c2_layer(x, w, live, group, rows, n, heads, dh, 1e-6)
    exp = _brute_layer(x, w, live, group, rows, n, heads, dh, 1e-6)
    assert oracle.rel_max_error(got, exp) <= 1e-5


def test_layer_with_zero_output_projections_is_identity(oracle):
    rows, n, heads, dh, d, dff = 3, 7, 2, 8, 16, 32
    w = _layer_weights(13, d, heads * dh, dff)
    for k in ("time_o", "group_o", "wo"):
        w[k] = np.zeros_like(w[k])
    x = _rng(14).standard_normal((rows * n, d)).astype(np.float32)
    live = np.ones((rows, n), np.int32)
    got = oracle.c2_layer(x, w, live, np.arange(rows, dtype=np.int32), rows, n, heads, dh, 1e-6)
    np.testing.assert_array_equal(got, x)
