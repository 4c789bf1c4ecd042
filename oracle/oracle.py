"""ctypes wrapper of libjc_oracle.so, the C restatement of the reference's CPU attention stages.

TEST INFRASTRUCTURE ONLY: the checker for libjitcast_hip. See jc_oracle.h for the reference
file:line each function restates.
"""
from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libjc_oracle.so"
_lib = None


def build() -> Path:
    if shutil.which("make") is None:
        raise RuntimeError("make is not available to build the oracle")
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ctypes.CDLL(str(LIB))
        v, i, f, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_int64
        sig = {
            "jco_c2_inv_freq": (None, [i, f, v]),
            "jco_c2_rope_table": (None, [i, i, f, v]),
            "jco_c2_time_attention": (i, [v, v, v, i, i, i, i, i, f, i]),
            "jco_c2_group_attention": (i, [v, v, v, v, i, i, i, i, i, i]),
            "jco_c2_live": (None, [v, i, i, i, i, i, v]),
            "jco_ts_inv_freq": (None, [i, i, f, v]),
            "jco_ts_time_attention": (i, [v, v, v, v, v, i, i, i, i, i, i, i, i, f, i]),
            "jco_ts_variate_attention": (i, [v, v, v, v, v, i, i, i, i, i, i, i, i]),
            "jco_ts_gate": (None, [v, v, i64]),
            "jco_linear": (None, [v, i, v, v, i, i, v, i]),
            "jco_rms_norm": (None, [v, i, i, v, f, v]),
            "jco_relu": (None, [v, i64]),
            "jco_add": (None, [v, v, i64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def _p(a: np.ndarray | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0) if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def c2_inv_freq(dh: int, theta: float = 10000.0) -> np.ndarray:
    out = np.empty(dh // 2, np.float32)
    lib().jco_c2_inv_freq(dh, theta, _p(out))
    return out


def c2_rope_table(n: int, dh: int, theta: float = 10000.0) -> np.ndarray:
    out = np.empty((n, dh), np.float32)
    lib().jco_c2_rope_table(n, dh, theta, _p(out))
    return out


def c2_time_attention(qkv, live, rows, n, heads, dh, inner, theta=10000.0, threads=0) -> np.ndarray:
    qkv, live = _f32(qkv), _i32(live)
    out = np.empty((rows * n, inner), np.float32)
    rc = lib().jco_c2_time_attention(_p(qkv), _p(out), _p(live), rows, n, heads, dh, inner, theta, threads)
    if rc:
        raise ValueError(f"jco_c2_time_attention: {rc}")
    return out


def c2_group_attention(qkv, live, group, rows, n, heads, dh, inner, threads=0) -> np.ndarray:
    qkv, live, group = _f32(qkv), _i32(live), _i32(group)
    out = np.empty((rows * n, inner), np.float32)
    rc = lib().jco_c2_group_attention(_p(qkv), _p(out), _p(live), _p(group), rows, n, heads, dh, inner, threads)
    if rc:
        raise ValueError(f"jco_c2_group_attention: {rc}")
    return out


def c2_live(window, rows, nc, patch, reg, h) -> np.ndarray:
    window = _f32(window)
    out = np.empty((rows, nc + reg + h), np.int32)
    lib().jco_c2_live(_p(window), rows, nc, patch, reg, h, _p(out))
    return out


def ts_inv_freq(dh: int, rope_dim: int, theta: float = 10000.0) -> np.ndarray:
    out = np.empty(dh // 2, np.float32)
    lib().jco_ts_inv_freq(dh, rope_dim, theta, _p(out))
    return out


def ts_time_attention(qkv, key_valid, known, pos, rows, enc, ll, n, heads, dh, d, rope_dim, theta=10000.0,
                      threads=0) -> np.ndarray:
    qkv, key_valid, known, pos = _f32(qkv), _i32(key_valid), _i32(known), _i32(pos)
    out = np.empty((rows * n, d), np.float32)
    rc = lib().jco_ts_time_attention(_p(qkv), _p(out), _p(key_valid), _p(known), _p(pos), rows, enc, ll, n, heads,
                                     dh, d, rope_dim, theta, threads)
    if rc:
        raise ValueError(f"jco_ts_time_attention: {rc}")
    return out


def ts_variate_attention(qkv, key_valid, group, role, covariates, rows, enc, n, heads, dh, d, threads=0):
    qkv, key_valid, group, role = _f32(qkv), _i32(key_valid), _i32(group), _i32(role)
    out = np.empty((rows * n, d), np.float32)
    rc = lib().jco_ts_variate_attention(_p(qkv), _p(out), _p(key_valid), _p(group), _p(role), int(covariates), rows,
                                        enc, n, heads, dh, d, threads)
    if rc:
        raise ValueError(f"jco_ts_variate_attention: {rc}")
    return out


def ts_gate(att, g) -> np.ndarray:
    att = _f32(att).copy()
    g = _f32(g)
    lib().jco_ts_gate(_p(att), _p(g), att.size)
    return att


def linear(x, w, b=None, threads=0) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    rows, inn = x.shape
    out_f = w.shape[0]
    y = np.empty((rows, out_f), np.float32)
    lib().jco_linear(_p(x), rows, _p(w), _p(None if b is None else _f32(b)), inn, out_f, _p(y), threads)
    return y


def rms_norm(x, w, eps) -> np.ndarray:
    x = _f32(x)
    rows, cols = x.shape
    y = np.empty_like(x)
    lib().jco_rms_norm(_p(x), rows, cols, _p(None if w is None else _f32(w)), eps, _p(y))
    return y


def relu(x) -> np.ndarray:
    y = _f32(x).copy()
    lib().jco_relu(_p(y), y.size)
    return y


def add(acc, x) -> np.ndarray:
    y = _f32(acc).copy()
    lib().jco_add(_p(y), _p(_f32(x)), y.size)
    return y


def c2_layer(x, w: dict, live, group, rows, n, heads, dh, eps, theta=10000.0, threads=0) -> np.ndarray:
    """One Chronos-2 encoder layer on x [rows*n, d], in the order CpuChronos2.forward runs it
    (CpuChronos2.java:150-161): rmsNorm, QKV, RoPE + time attention, O, residual add; the same for
    group attention; rmsNorm, Wi, ReLU, Wo, residual add. w holds numpy arrays keyed like
    jc_c2_layer_weights (biases optional)."""
    inner = heads * dh
    x = _f32(x)
    hn = rms_norm(x, w["time_norm"], eps)
    qkv = linear(hn, w["time_qkv"], w.get("time_qkv_bias"), threads)
    att = c2_time_attention(qkv, live, rows, n, heads, dh, inner, theta, threads)
    x = add(x, linear(att, w["time_o"], w.get("time_o_bias"), threads))
    hn = rms_norm(x, w["group_norm"], eps)
    qkv = linear(hn, w["group_qkv"], w.get("group_qkv_bias"), threads)
    att = c2_group_attention(qkv, live, group, rows, n, heads, dh, inner, threads)
    x = add(x, linear(att, w["group_o"], w.get("group_o_bias"), threads))
    hn = rms_norm(x, w["mlp_norm"], eps)
    act = relu(linear(hn, w["wi"], w.get("wi_bias"), threads))
    return add(x, linear(act, w["wo"], w.get("wo_bias"), threads))


def c2_residual(x, w: dict, prefix: str, threads=0) -> np.ndarray:
    """CpuChronos2.Residual.apply (CpuChronos2.java:57-69): output(ReLU(hidden(x))) + residual(x)."""
    h = relu(linear(x, w[prefix + "_hidden_w"], w.get(prefix + "_hidden_b"), threads))
    y = linear(h, w[prefix + "_output_w"], w.get(prefix + "_output_b"), threads)
    return add(y, linear(x, w[prefix + "_residual_w"], w.get(prefix + "_residual_b"), threads))


def c2_forward_raw(tokens, w: dict, live, group, rows, nc, nreg, h, heads, dh, eps, theta=10000.0,
                   threads=0, sink=None) -> np.ndarray:
    """CpuChronos2.forward from the patch tokens to the raw output patch embedding
    (CpuChronos2.java:122-169): the input embedding, the context / [REG] / future token order, the
    encoder layers, the final RMSNorm, the future tokens, the output embedding. tokens
    [rows*(nc+h), 3P]; w as jitcast_amd.chronos2_model.random_weights lays it out."""
    ne, n = nc + h, nc + nreg + h
    emb = c2_residual(tokens, w, "in", threads)
    d = emb.shape[1]
    x = np.empty((rows * n, d), np.float32)
    for i in range(rows):
        x[i * n: i * n + nc] = emb[i * ne: i * ne + nc]
        if nreg:
            x[i * n + nc] = w["shared"][1]
        x[i * n + nc + nreg: (i + 1) * n] = emb[i * ne + nc: (i + 1) * ne]
    for li, lw in enumerate(w["layers"]):
        x = c2_layer(x, lw, live, group, rows, n, heads, dh, eps, theta, threads)
        if sink is not None:
            sink(f"layer{li}", x)
    y = rms_norm(x, w["final_norm"], eps)
    dec = np.concatenate([y[i * n + nc + nreg: (i + 1) * n] for i in range(rows)])
    return c2_residual(dec, w, "out", threads)


def c2_model_forward(c, w: dict, context, group, future, output_patches, threads=0, sink=None) -> np.ndarray:
    """CpuChronos2.forward(ModelInput) (CpuChronos2.java:122-173) end to end on the oracle's pieces:
    ModelLayout.of's window (the last context_length steps, NaN-padded on the left to whole patches),
    future covariates and live mask (ModelLayout.java:70-116), ModelPrep.of, the forward and
    ModelPrep.finish. context [rows][T] (equal lengths), group [rows] (any ids, rows of a group need
    not be adjacent), future [rows][<= output_patches*P] or None. `c` carries the config fields
    (patch_size, context_length, use_reg_token, num_heads, d_kv, layer_norm_eps, rope_theta,
    time_encoding_scale, use_arcsinh, quantiles). sink(name, x) sees each layer's output, as the
    reference's StageSink. Returns [rows][Q][output_patches*P]."""
    ps, h = c.patch_size, int(output_patches)
    if h < 1:
        raise ValueError(f"output patches must be >= 1, got {h}")
    ctx = np.asarray(context, np.float32)
    rows, t = ctx.shape
    group = _i32(group)
    if group.shape != (rows,):
        raise ValueError("group ids must have one entry per row")
    kept = min(t, c.context_length)
    padded = (kept + ps - 1) // ps * ps
    nc = padded // ps
    window = np.full((rows, padded), np.nan, np.float32)
    window[:, padded - kept:] = ctx[:, t - kept:]
    fut = np.full((rows, h * ps), np.nan, np.float32)
    if future is not None:
        for i in range(rows):
            f = np.asarray(future[i], np.float32)
            if f.size > h * ps:
                raise ValueError(f"{h} output patches cannot hold {f.size} future steps")
            fut[i, : f.size] = f
    nreg = 1 if c.use_reg_token else 0
    live = c2_live(window, rows, nc, ps, nreg, h)
    tok, loc, scale = c2_prep(window, fut, nc, h, ps, c.time_encoding_scale, c.use_arcsinh)
    raw = c2_forward_raw(tok, w, live, group, rows, nc, nreg, h, c.num_heads, c.d_kv, c.layer_norm_eps, c.rope_theta,
                         threads, sink=sink)
    return c2_finish(raw, loc, scale, rows, h, len(c.quantiles), ps, c.use_arcsinh)


def silu(x) -> np.ndarray:
    """Ops.silu (J/cpu/Ops.java:68-70): (float) (v / (1.0 + exp(-v))), in double, rounded."""
    v = _f32(x).astype(np.float64)
    return (v / (1.0 + np.exp(-v))).astype(np.float32)


def swiglu(up, f: int) -> np.ndarray:
    """CpuTimestral.s MLP activation (CpuTimestral.java:165-172): act[t][j] = silu(up[t][j]) *
    up[t][f + j], the product in float."""
    up = _f32(up)
    return silu(up[:, :f]) * up[:, f:2 * f]


def ts_residual(x, w: dict, prefix: str, threads=0) -> np.ndarray:
    """CpuTimestral.Residual.apply (CpuTimestral.java:58-71): output(SiLU(hidden(x))) + residual(x)."""
    h = silu(linear(x, w[prefix + "_hidden_w"], w.get(prefix + "_hidden_b"), threads))
    y = linear(h, w[prefix + "_output_w"], w.get(prefix + "_output_b"), threads)
    return add(y, linear(x, w[prefix + "_residual_w"], w.get(prefix + "_residual_b"), threads))


def ts_forward_raw(tokens, w: dict, key_valid, known, position, group, role, covariates, rows, enc, ll, h, heads,
                   dh, rope_dim, eps, theta=10000.0, threads=0) -> np.ndarray:
    """CpuTimestral.predictBlock from the patch tokens to the head's raw outputs
    (CpuTimestral.java:127-188): the patch embedding, the encoder tokens then h forecast-query tokens
    per row, per layer each attention sublayer (rmsNorm, q|k|v, time attention with RoPE at
    `position` or variate attention, the sigmoid gate, the output projection added) and the SwiGLU
    MLP, the output norm, the decoder tokens, the head. tokens [rows*enc, 2P]; w as
    jitcast_amd.timestral_model.random_weights lays it out; returns [rows*h, P*Q]."""
    n = enc + h
    emb = ts_residual(tokens, w, "embed", threads)
    d = emb.shape[1]
    x = np.empty((rows * n, d), np.float32)
    for i in range(rows):
        x[i * n: i * n + enc] = emb[i * enc: (i + 1) * enc]
        x[i * n + enc: (i + 1) * n] = _f32(w["query"])
    x = ts_encoder(x, w, key_valid, known, position, group, role, covariates, rows, enc, ll, h, heads, dh, rope_dim,
                   eps, theta, threads)
    y = rms_norm(x, w["out_norm"], eps)
    dec = np.concatenate([y[i * n + enc: (i + 1) * n] for i in range(rows)])
    return ts_residual(dec, w, "head", threads)


def ts_encoder(x, w: dict, key_valid, known, position, group, role, covariates, rows, enc, ll, h, heads, dh, rope_dim,
               eps, theta=10000.0, threads=0, mlp=True) -> np.ndarray:
    """CpuTimestral.predictBlock's layer loop (CpuTimestral.java:150-172) on x [rows*(enc+h), d]:
    per layer each attention sublayer (rmsNorm, q|k|v, time attention with RoPE at `position` or
    variate attention, the sigmoid gate, the output projection added), then the SwiGLU MLP unless
    mlp is False (the attention-only stack). Returns the new x."""
    n = enc + h
    d = x.shape[1]
    x = _f32(x)
    for lw in w["layers"]:
        for a in lw["attentions"]:
            hn = rms_norm(x, a["norm"], eps)
            qkv = linear(hn, a["qkv"], None, threads)
            if a["time"]:
                att = ts_time_attention(qkv, key_valid, known, position, rows, enc, ll, n, heads, dh, d, rope_dim, theta,
                                        threads)
            else:
                att = ts_variate_attention(qkv, key_valid, group, role, covariates, rows, enc, n, heads, dh, d, threads)
            if a.get("gate") is not None:
                att = ts_gate(att, linear(hn, a["gate"], None, threads))
            x = add(x, linear(att, a["wo"], None, threads))
        if not mlp:
            continue
        hn = rms_norm(x, lw["mlp_norm"], eps)
        f = lw["down"].shape[1]
        act = swiglu(linear(hn, lw["up"], None, threads), f)
        x = add(x, linear(act, lw["down"], None, threads))
    return x


def ts_block_prep(window, observed, known, patch, minimum_scale, use_asinh):
    """BlockPrep.of (J/timestral/BlockPrep.java:40-75) value by value: Scaler.causalPatchLocScale
    (Scaler.java:40-64) for every row, Scaler.instanceNorm (Scaler.java:87-110) for known covariate
    rows (arcsinh off for a binary one), Scaler.affine (Scaler.java:73-79). Returns (tokens
    [rows*enc, 2P], scaled, loc, scale [rows, w])."""
    window = _f32(window)
    rows, w = window.shape
    enc = w // patch
    f32 = np.float32
    ms = float(f32(minimum_scale))
    eps = float(np.finfo(np.float32).eps)
    loc = np.zeros((rows, w), f32)
    scale = np.zeros((rows, w), f32)
    scaled = np.zeros((rows, w), f32)
    tok = np.zeros((rows * enc, 2 * patch), f32)
    for i in range(rows):
        cw = cx = m2 = prev = 0.0
        for t in range(w):
            wt = 1.0 if observed[i][t] else 0.0
            xi = float(window[i][t])
            cw += wt
            cx += wt * xi
            mean = cx / max(cw, 1.0)
            m2 += (xi - prev) * (xi - mean) * wt
            prev = mean
            if t % patch == patch - 1:
                var = m2 / max(max(cw, 1.0) - 1.0, 1.0)
                for j in range(t - patch + 1, t + 1):
                    loc[i][j] = f32(mean)
                    scale[i][j] = f32(max(float(np.sqrt(var)), ms))
        asinh = use_asinh
        if known[i]:
            n = 0.0
            total = 0.0
            zero_one, anyo = True, False
            for t in range(w):
                if observed[i][t]:
                    n += 1
                    total += float(window[i][t])
                    anyo = True
                zero_one = zero_one and (window[i][t] == 0 or window[i][t] == 1 or not observed[i][t])
            n = max(n, 1.0)
            lo = f32(total / n)
            ss = 0.0
            for t in range(w):
                dv = f32(window[i][t] - lo) if observed[i][t] else f32(0)
                ss += float(dv) * float(dv)
            sc = max(f32(np.sqrt(float(f32(ss / n)))), f32(ms))
            if zero_one and anyo:
                lo, sc = f32(0), f32(1)
                asinh = False
            loc[i][:] = lo
            scale[i][:] = sc
        for t in range(w):
            if not observed[i][t]:
                continue
            v = f32(f32(window[i][t] - loc[i][t]) / max(scale[i][t], f32(eps)))
            if asinh:
                a = abs(float(v))
                r = np.log(a + np.sqrt(a * a + 1.0))
                v = f32(-r if v < 0 else r)
            scaled[i][t] = v
        for p in range(enc):
            for s in range(patch):
                tok[i * enc + p][s] = scaled[i][p * patch + s]
                tok[i * enc + p][patch + s] = f32(0) if observed[i][p * patch + s] else f32(1)
    return tok, scaled, loc, scale


def ts_quantile_map(raw, knots, median, width_factor):
    """Quantiles.apply (J/timestral/Quantiles.java:52-77) on each row of raw [..., Q], in place order:
    levels above the median from the median up, below it from the median down."""
    raw = _f32(raw).reshape(-1, len(knots)).copy()
    f32 = np.float32
    q = len(knots)
    width = [f32(f32(width_factor) * f32(knots[i] - knots[i - 1] if i > median else knots[i + 1] - knots[i]
                                          if i < median else 0.0)) for i in range(q)]
    big = float(np.finfo(np.float32).max)

    def softplus(x):
        return x if x > 20 else f32(np.log1p(np.exp(float(x))))

    for row in raw:
        m = row[median]
        up = f32(0)
        for i in range(median + 1, q):
            up = f32(up + f32(width[i] * softplus(row[i])))
            row[i] = f32(min(max(float(f32(m + up)), -big), big))
        down = f32(0)
        for i in range(median - 1, -1, -1):
            down = f32(down + f32(width[i] * softplus(row[i])))
            row[i] = f32(min(max(float(f32(m - down)), -big), big))
        row[median] = f32(min(max(float(m), -big), big))
    return raw


def ts_block_finish(raw, loc, scale, ll, h, patch, knots, median, width_factor, use_asinh):
    """BlockPrep.finish (J/timestral/BlockPrep.java:77-101) value by value: the quantile map on every
    step's Q raw values, Scaler.invert with the loc/scale of the last context patch's first step
    (sinh when use_asinh; float multiply, then add), Scaler.clampNonFinite (Scaler.java:118-130) per
    step. raw [rows*h, P*Q]; returns [rows, h*P, Q]."""
    rows = np.asarray(loc).shape[0]
    q = len(knots)
    f32 = np.float32
    v = ts_quantile_map(np.asarray(raw, np.float32).reshape(rows * h * patch, q), knots, median, width_factor)
    v = v.reshape(rows, h * patch, q)
    out = np.zeros_like(v)
    for i in range(rows):
        a_loc, a_scale = f32(loc[i][(ll - 1) * patch]), f32(scale[i][(ll - 1) * patch])
        for t in range(h * patch):
            vals = []
            for k in range(q):
                x = v[i][t][k]
                with np.errstate(over="ignore"):
                    x = f32(np.sinh(float(x))) if use_asinh else x
                vals.append(f32(f32(x * a_scale) + a_loc))
            fin = [x for x in vals if np.isfinite(x)]
            hi = max(fin) if fin else -np.inf
            lo = min(fin) if fin else np.inf
            for k, x in enumerate(vals):
                y = hi if x == np.inf else lo if x == -np.inf else x
                out[i][t][k] = f32(0) if np.isinf(y) else y
    return out


def c2_instance_norm(row) -> tuple:
    """ModelPrep.instanceNorm (ModelPrep.java:80-101), value by value: mean and population std of the
    observed values in double, rounded to float; a zero std floored at 1e-5; (0, 1) with none."""
    total, cnt = 0.0, 0
    for v in row:
        if not np.isnan(v):
            total += float(v)
            cnt += 1
    if cnt == 0:
        return np.float32(0), np.float32(1)
    loc = np.float32(total / cnt)
    ss = 0.0
    for v in row:
        if not np.isnan(v):
            dv = np.float32(np.float32(v) - loc)
            ss += float(dv) * float(dv)
    scale = np.float32(np.sqrt(ss / cnt))
    return loc, (np.float32(1e-5) if scale == 0 else scale)


def _c2_scaled(v, loc, scale, arcsinh):
    """ModelPrep.scaled / asinh (ModelPrep.java:104-114)."""
    x = np.float32(np.float32(np.float32(v) - loc) / scale)
    if not arcsinh:
        return x
    a = abs(float(x))
    r = np.log(a + np.sqrt(a * a + 1.0))
    return np.float32(-r if x < 0 else r)


def c2_prep(window, future, nc, h, patch, time_scale, arcsinh):
    """ModelPrep.of (ModelPrep.java:38-72), row by row: tokens [rows*(nc+h), 3P] of time encoding,
    scaled value (0 where missing) and observation mask; loc, scale [rows]."""
    rows = window.shape[0]
    ps, ne = patch, nc + h
    tok = np.zeros((rows * ne, 3 * ps), np.float32)
    loc = np.zeros(rows, np.float32)
    scale = np.zeros(rows, np.float32)
    for i in range(rows):
        loc[i], scale[i] = c2_instance_norm(window[i])
        for p in range(ne):
            for s in range(ps):
                if p < nc:
                    t = p * ps + s
                    te, v = np.float32(np.float32(t - nc * ps) / np.float32(time_scale)), window[i][t]
                else:
                    t = (p - nc) * ps + s
                    te, v = np.float32(np.float32(t) / np.float32(time_scale)), future[i][t]
                obs = not np.isnan(v)
                tok[i * ne + p, s] = te
                tok[i * ne + p, ps + s] = _c2_scaled(v, loc[i], scale[i], arcsinh) if obs else np.float32(0)
                tok[i * ne + p, 2 * ps + s] = 1.0 if obs else 0.0
    return tok, loc, scale


def c2_finish(raw, loc, scale, rows, h, q, patch, arcsinh) -> np.ndarray:
    """ModelPrep.finish (ModelPrep.java:125-150): [rows, Q, h*P] = sinh(raw)*scale + loc."""
    out = np.zeros((rows, q, h * patch), np.float32)
    for i in range(rows):
        for p in range(h):
            for k in range(q):
                for s in range(patch):
                    v = np.float32(raw[i * h + p, k * patch + s])
                    if arcsinh:
                        v = np.float32(np.sinh(float(v)))
                    out[i, k, p * patch + s] = np.float32(np.float32(v * scale[i]) + loc[i])
    return out


def rel_max_error(actual, expected) -> float:
    """The reference's metric: max|a-e| / max(max|e|, 1e-6); a NaN mismatch is infinite
    (T/chronos2/Chronos2Golden.java:218-234)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    if a.shape != e.shape:
        raise ValueError(f"shape {a.shape} vs {e.shape}")
    if a.size == 0:
        return 0.0
    an, en = np.isnan(a), np.isnan(e)
    if np.any(an != en):
        return float("inf")
    d = np.abs(np.where(an, 0, a) - np.where(en, 0, e))
    scale = max(float(np.max(np.abs(np.where(en, 0, e)))), 1e-6)
    return float(np.max(d)) / scale


def ts_block_layout(inputs, observed, group, h, patch, role=None, known_future=None, known_future_mask=None,
                    covariate_enabled=True, attend_missing=True, block_size=64):
    """BlockLayout.of (J/timestral/BlockLayout.java:77-148) and position() (203-207), row by row:
    the window (the context, plus the horizon's known-future steps when some row is a covariate),
    keyValid per encoder patch (observed, or with attend_missing any patch from the row's first
    observed one on), the first patch any row of the series observes (0 if none), known rows. Returns
    (window [rows, enc*P], window_observed, enc, covariates, key_valid [rows, enc] int32, known [rows]
    int32, position [rows, enc+h] int32, ll). ValueError as BlockLayout.of's IllegalArgumentExceptions."""
    x = np.asarray(inputs, np.float32)
    obs_in = np.asarray(observed, bool)
    rows, t = x.shape
    if t % patch:
        raise ValueError(f"context length {t} is not a multiple of the patch size {patch}")
    if h < 1:
        raise ValueError(f"horizon patches must be >= 1, got {h}")
    cov = False
    if role is not None and covariate_enabled:
        for v in role:
            cov = cov or int(v) != 0
    ll = t // patch
    window, wobs = x, obs_in
    roles = [0] * rows
    if cov:
        if h > block_size:
            raise ValueError(f"a block with covariates decodes at most {block_size} patches, got {h}")
        roles = [int(v) for v in role]
        window = np.zeros((rows, t + h * patch), np.float32)
        wobs = np.zeros((rows, t + h * patch), bool)
        for i in range(rows):
            window[i, :t] = x[i]
            wobs[i, :t] = obs_in[i]
            if known_future is not None:
                window[i, t:] = np.asarray(known_future[i], np.float32)[: h * patch]
                wobs[i, t:] = np.asarray(known_future_mask[i], bool)[: h * patch]
    enc = window.shape[1] // patch
    valid = np.zeros((rows, enc), np.int32)
    patch_obs = np.zeros((rows, enc), bool)
    for i in range(rows):
        started = False
        for p in range(enc):
            anyo = False
            for s in range(p * patch, (p + 1) * patch):
                anyo = anyo or bool(wobs[i][s])
            patch_obs[i][p] = anyo
            started = started or anyo
            valid[i][p] = 1 if (started if attend_missing else anyo) else 0
    group_first = {}
    for i in range(rows):
        f = enc
        for p in range(enc):
            if patch_obs[i][p]:
                f = p
                break
        g = int(group[i])
        group_first[g] = min(group_first.get(g, f), f)
    position = np.zeros((rows, enc + h), np.int32)
    for i in range(rows):
        f = group_first[int(group[i])]
        first = 0 if f == enc else f
        for k in range(enc + h):
            position[i][k] = (k if k < enc else ll + k - enc) - first
    known = np.array([1 if cov and roles[i] == 2 else 0 for i in range(rows)], np.int32)
    return window, wobs, enc, cov, valid, known, position, ll
