"""Headline benchmark: fused Chronos-2 fp32 time attention at L=513, 12x64 heads, on one MI355X.

One step is one launch of jc_c2_time_attention over the whole config-1 batch (B=256 series,
L=513, 12 heads x 64; RoPE at load; left padding U{0..256} masked), inputs resident in HBM. The
value is mask-aware TFLOP/s: sum over (series, head, query) of 4*dh*|live keys| per step, divided
by the step time. The roofline object prices the kernel's average launch time (HIP events on the
launch stream) against the fp32 MFMA peak; the CPU baseline is the C oracle (a restatement of the
reference's CPU engine) timed on a bounded sample of the same workload on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PEAK_FP32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0
METRIC = "fused attention TFLOP/s (% MFMA peak) at L=513, 12x64 heads; forecast series/sec"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def traffic_from_profile(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by a
    known-size copy), committed as profiles/<name>.traffic.json; None when not measured."""
    p = ROOT / "profiles" / f"{name}.traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("bytes_per_launch")
    except Exception:
        return None


def cpu_baseline(case, sample_rows: int, threads: int):
    """Times the oracle (C restatement of CpuChronos2.timeAttention) on the first sample_rows rows."""
    import numpy as np

    sys.path.insert(0, str(ROOT))
    from oracle import oracle

    rows, n, heads, dh, inner = sample_rows, case.n, case.heads, case.dh, case.inner
    qkv = case.qkv[: rows * n].float().cpu().numpy()
    live = case.live[: rows * n].cpu().numpy().astype(np.int32)
    oracle.lib()
    t0 = time.perf_counter()
    oracle.c2_time_attention(qkv, live, rows, n, heads, dh, inner, threads=threads)
    dt = time.perf_counter() - t0
    flops = 4.0 * dh * heads * n * float(live.sum())
    return {
        "value": round(flops / dt / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{rows} of {case.rows} series of config 1 (L={n}, {heads}x{dh}), mask-aware flops, "
                  f"{dt:.2f} s, double accumulation",
    }


def time_launches(fn, steps: int, warmup: int):
    """Average launch time (ms) over `steps` launches, HIP events on the launch stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in ev) / len(ev)


def group_attention_line(steps: int, warmup: int) -> dict:
    """Config 2: fp32 group attention, 4096 rows x 129 slots, groups U{1..64}; HBM-bound."""
    import torch

    from jitcast_amd import chronos2, synthetic

    case = synthetic.c2_group_config2(device="cuda")
    out = torch.empty(case.rows * case.n, case.inner, dtype=torch.float32, device="cuda")

    def fn():
        chronos2.group_attention(case.qkv, out, case.live, case.group_start, case.group_end, case.rows, case.n,
                                 case.heads, case.dh, case.inner)

    ms = time_launches(fn, steps, warmup)
    nbytes = case.algorithmic_bytes()
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"group attention: {ms:.4f} ms, {gbs:.0f} GB/s algorithmic ({100 * gbs / PEAK_HBM_GBS:.1f}% of HBM)")
    res = {
        "workload": "config 2: fp32 Chronos-2 group attention, 4096 rows x 129 slots, 12x64, groups U{1..64}",
        "kernel": "jc::group_attention_f32<64, false, true>",
        "launch_ms": round(ms, 5),
        "value": round(gbs, 1),
        "unit": "GB/s",
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic_from_profile("c2_group_attention_f32_config2")},
        "bytes_per_launch": nbytes,
        "tflops": round(case.flops() / (ms * 1e-3) / 1e12, 2),
    }
    del case, out
    torch.cuda.empty_cache()
    return res


def time_attention_lowp_line(case, steps: int, warmup: int, dtype_name: str) -> dict:
    """Config 1-bf16 (or fp16): the config-1 inputs with qkv rounded to the storage type (what a
    projection epilogue writing bf16 hands over); fp32 accumulation and softmax."""
    import torch

    from jitcast_amd import chronos2

    dt = {"bf16": torch.bfloat16, "fp16": torch.float16}[dtype_name]
    q16 = case.qkv.to(dt)
    out = torch.empty(case.rows * case.n, case.inner, dtype=dt, device=q16.device)

    def fn():
        chronos2.time_attention(q16, out, case.live, case.rows, case.n, case.heads, case.dh, case.inner, case.table)

    ms = time_launches(fn, steps, warmup)
    flops = case.mask_aware_flops()
    tf = flops / (ms * 1e-3) / 1e12
    log(f"time attention {dtype_name}: {ms:.4f} ms, {tf:.1f} TFLOP/s mask-aware "
        f"({100 * tf / PEAK_BF16_TFLOPS:.1f}% of the {dtype_name} MFMA peak)")
    res = {
        "workload": f"config 1-{dtype_name}: the config-1 inputs with qkv in {dtype_name}, fp32 accumulation",
        "kernel": "jc::time_attention_lpp<%s, true>" % {"bf16": "__bf16", "fp16": "_Float16"}[dtype_name],
        "launch_ms": round(ms, 5),
        "value": round(tf, 2),
        "unit": "TFLOP/s",
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profile(f"c2_time_attention_{dtype_name}_config1")},
        "dense_tflops": round(case.dense_flops() / (ms * 1e-3) / 1e12, 2),
    }
    del q16, out
    torch.cuda.empty_cache()
    return res


def layer_line(steps: int, warmup: int, dtype_name: str = "f32") -> dict:
    """Config 4's encoder-layer shape through jc_c2_layer: RMSNorm, the six GEMMs of the layer, RoPE
    time attention, group attention, ReLU and the residual adds. f32: everything fp32. bf16: the
    GEMMs and the time attention in bf16 with fp32 accumulation (weights converted once, outside the
    timed region), the group attention, norms and residual stream fp32."""
    import torch

    from jitcast_amd import _lib, chronos2, synthetic

    case = synthetic.c2_layer_config4(device="cuda")
    code = {"f32": _lib.JC_F32, "bf16": _lib.JC_BF16}[dtype_name]
    weights = dict(case.weights)
    ws = case.workspace
    if code != _lib.JC_F32:
        for k in ("time_qkv", "time_o", "group_qkv", "group_o", "wi", "wo"):
            lp = torch.empty(weights[k].shape, dtype=torch.bfloat16, device="cuda")
            chronos2.to_lp(weights[k], lp)
            weights[k] = lp
        inner = case.heads * case.dh
        ws = torch.empty(chronos2.layer_workspace_bytes(case.rows, case.n, case.d, inner, case.dff, code) // 4 + 64,
                         dtype=torch.float32, device="cuda")
    x0 = case.x.clone()

    def fn():
        chronos2.layer(case.x, weights, case.live, case.table, case.group_start, case.group_end, ws, case.rows,
                       case.n, case.d, case.heads, case.dh, case.dff, 1e-6, code)

    ms = time_launches(fn, steps, warmup)
    case.x.copy_(x0)
    flops = case.flops()
    tf = flops / (ms * 1e-3) / 1e12
    peak = PEAK_FP32_TFLOPS if code == _lib.JC_F32 else PEAK_BF16_TFLOPS
    tokens = case.rows * case.n
    log(f"layer {dtype_name}: {ms:.3f} ms, {tf:.1f} TFLOP/s ({100 * tf / peak:.1f}% of the {dtype_name} MFMA peak), "
        f"{tokens / (ms * 1e-3) / 1e6:.1f} M tokens/s")
    res = {
        "workload": f"config 4 encoder-layer shape: 1024 groups x (4 series + 1 known covariate), 133 tokens "
                    f"(128 context patches + REG + 4 future), d_model 768, 12x64, d_ff 3072, {dtype_name}",
        "kernel": "jc_c2_layer (%s for the GEMMs)" % ("jc::gemm_f32" if code == _lib.JC_F32 else "jc::gemm_lp<__bf16>"),
        "launch_ms": round(ms, 4),
        "value": round(tf, 2),
        "unit": "TFLOP/s",
        "tokens_per_s": round(tokens / (ms * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tf / peak, 4),
                     "traffic": traffic_from_profile(f"c2_layer_{dtype_name}_config4")},
        "flops_per_step": flops,
        "gemm_share_of_flops": round(case.gemm_flops() / flops, 4),
    }
    del case, x0, weights, ws
    torch.cuda.empty_cache()
    return res


def ts_time_attention_line(steps: int, warmup: int) -> dict:
    """Config 3's attention stack: the bf16 Timestral time attention (RoPE, mask, fused gate) of 12
    layers per step on 64 series x 1024 tokens, 12 x 64 heads."""
    import torch

    from jitcast_amd import synthetic, timestral

    case = synthetic.ts_time_config3(device="cuda")
    out = torch.empty(case.rows * case.n, case.d, dtype=torch.bfloat16, device="cuda")
    layers = 12

    def fn():
        for _ in range(layers):
            timestral.time_attention(case.qkv, out, case.key_valid, case.known, case.pos, case.table, case.gate,
                                     case.rows, case.n, case.n, case.n, case.heads, case.dh, case.d)

    ms = time_launches(fn, steps, warmup)
    flops = layers * case.mask_aware_flops()
    tf = flops / (ms * 1e-3) / 1e12
    log(f"config 3 attention stack bf16: {ms:.3f} ms for {layers} layers, {tf:.1f} TFLOP/s mask-aware "
        f"({100 * tf / PEAK_BF16_TFLOPS:.1f}% of the bf16 MFMA peak)")
    res = {
        "workload": "config 3: Timestral time attention in bf16 (RoPE on half the head, bidirectional over valid "
                    "keys, left padding U{0..256}, fused gate), 64 series x 1024 tokens, 12x64, 12 layers per step",
        "kernel": "jc::time_attention_lp<__bf16, 64, 4, true, true, true>",
        "launch_ms": round(ms / layers, 5),
        "value": round(tf, 2),
        "unit": "TFLOP/s",
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None},
    }
    del case, out
    torch.cuda.empty_cache()
    return res


def forecast_line(steps: int, warmup: int, dtype_name: str = "f32") -> dict:
    """Config 4 end to end: HipChronos2Model.forecast on 1024 groups x (4 series + 1 known-future
    covariate) of 2048 steps, horizon 64, 21 quantiles, Chronos-2 120M-class random-init weights.
    value = target series forecast per second, wall clock around forecast() (the group order on the
    host, one upload, jc_c2_prep, the device forward launched kernel by kernel, jc_c2_finish, one
    download). The same forecast with the forward replayed from its plan (max_plans: one hipGraph
    per shape, as the reference's forward runs from its PlanCache) is timed beside it, at config 4
    and on a 20-row request."""
    import numpy as np
    import torch

    from jitcast_amd import chronos2_model as cm, synthetic

    c = cm.Chronos2Config()  # d_model 768, 12 x 64, 12 layers, d_ff 3072, patch 16, 21 quantiles
    w = cm.random_weights(c, seed=0)
    model = cm.HipChronos2Model(c, w, dtype=dtype_name)
    planned = cm.HipChronos2Model(c, w, dtype=dtype_name, max_plans=1)
    del w
    ctx, group, fut, targets = synthetic.c2_forecast_config4()
    h = 64 // c.patch_size

    def timed(m):
        for _ in range(warmup):
            m.forecast(ctx, group, fut, h=h)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            o = m.forecast(ctx, group, fut, h=h)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps, o

    wall, out = timed(model)
    plan_wall, plan_out = timed(planned)
    assert np.array_equal(out, plan_out)
    # a small request (4 groups = 20 rows, 512 steps), where launching ~200 kernels from the host
    # costs more than the device work
    small = (ctx[:20, -512:], group[:20], fut[:20] if fut is not None else None)
    lat = {}
    for name, m in (("eager", model), ("plan", planned)):
        for _ in range(3):
            m.forecast(*small, h=h)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(20):
            m.forecast(*small, h=h)
        torch.cuda.synchronize()
        lat[name] = (time.perf_counter() - t0) / 20 * 1e3
    planned.close()
    del planned
    # the device forward alone (prepared tokens resident), HIP events
    lay = cm.layout(c, ctx, group, fut, h)
    tok, _, _ = cm.prep(c, lay)
    gs, ge = cm.chronos2.group_bounds(lay.group)
    dev = model.dev
    args = (torch.from_numpy(tok).to(dev), torch.from_numpy(lay.live.reshape(-1)).to(dev), torch.from_numpy(gs).to(dev),
            torch.from_numpy(ge).to(dev), lay.rows, lay.nc, lay.h)
    dev_ms = time_launches(lambda: model.forward_raw(*args), max(2, steps), 1)
    series = int(targets.sum())
    assert np.isfinite(out).all()
    log(f"forecast {dtype_name}: {wall * 1e3:.1f} ms per call end to end ({series / wall:.0f} series/s; from the "
        f"plan {plan_wall * 1e3:.1f} ms, {series / plan_wall:.0f} series/s), device forward "
        f"{dev_ms:.1f} ms ({series / (dev_ms * 1e-3):.0f} series/s); 20-row request {lat['plan']:.2f} ms from the "
        f"plan, {lat['eager']:.2f} ms eager")
    res = {
        "workload": f"config 4: Chronos-2 120M-class forecast ({dtype_name} encoder), 1024 groups x (4 series + 1 "
                    "known-future covariate) x 2048 steps, horizon 64, 21 quantiles, random-init weights",
        "metric": "forecast series/sec",
        "value": round(series / wall, 1),
        "unit": "series/s",
        "ms_per_call": round(wall * 1e3, 2),
        "plan_ms_per_call": round(plan_wall * 1e3, 2),
        "plan_series_per_s": round(series / plan_wall, 1),
        "small_request_ms": {"rows": 20, "steps": 512, "plan": round(lat["plan"], 3), "eager": round(lat["eager"], 3)},
        "device_forward_ms": round(dev_ms, 2),
        "device_series_per_s": round(series / (dev_ms * 1e-3), 1),
        "rows": lay.rows, "tokens_per_row": lay.n,
    }
    del model
    torch.cuda.empty_cache()
    return res


def ts_block_line(steps: int, warmup: int, dtype_name: str = "f32") -> dict:
    """The Timestral block end to end at config 3's shape: HipTimestralModel.predict_block on 64
    univariate series of 1023 patches (16,368 steps, left padding U{0..256} patches unobserved) and
    one forecast patch, 1024 tokens per series, a 123M-class model (d_model 768, 12 x 64, 12 layers
    of time + variate attention with gates, SwiGLU MLP 3072), random-init weights; fp32 or the
    FP16-GEMM mode in bf16.
    value = series per second, wall clock around predict_block (BlockLayout's window on the host,
    then BlockPrep, the forward and finish on the device, the quantiles copied back); the device
    forward alone timed with HIP events."""
    import numpy as np
    import torch

    from jitcast_amd import rng, timestral
    from jitcast_amd import timestral_model as tm

    c = tm.TimestralConfig()
    model = tm.HipTimestralModel(c, tm.random_weights(c, seed=0), dtype=dtype_name)
    rows, patches, h = 64, 1023, 1
    t = patches * c.patch_size
    x = rng.normal(rng.stream_seed(3, 0), rows * t, 1.0).reshape(rows, t).astype(np.float32)
    pad = rng.randint(rng.stream_seed(3, 1), rows, 0, 256)
    obs = np.arange(t)[None, :] >= (pad * c.patch_size)[:, None]
    group = np.arange(rows, dtype=np.int32)
    for _ in range(warmup):
        model.predict_block(x, obs, group, h)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = model.predict_block(x, obs, group, h)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    enc, _, kv, known, pos = timestral.block_layout(obs, group, h, c.patch_size)
    tok, _, _, _ = tm.block_prep(c, x, obs, known)
    gs, ge = tm.chronos2.group_bounds(group)
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(model.dev)  # noqa: E731
    args = (up(tok), up(kv.reshape(-1)), up(known), up(pos.reshape(-1)), up(gs), up(ge), None, False, rows, enc, h)
    dev_ms = time_launches(lambda: model.forward_raw(*args), max(2, steps), 1)
    assert np.isfinite(out).all()
    n = enc + h
    d, f = c.d_model, c.mlp_hidden_dim
    gemm_flops = 2.0 * rows * n * len(c.layers) * (2 * 5 * d * d + 3 * f * d)
    log(f"ts block {dtype_name}: {wall * 1e3:.1f} ms per predict_block ({rows / wall:.0f} series/s), device forward "
        f"{dev_ms:.1f} ms ({rows / (dev_ms * 1e-3):.0f} series/s, GEMMs {gemm_flops / (dev_ms * 1e-3) / 1e12:.1f} TFLOP/s)")
    res = {
        "workload": f"config 3 shape: Timestral 123M-class block forward ({dtype_name}), 64 univariate series x 1023 patches "
                    "+ 1 forecast patch (1024 tokens), left padding U{0..256} patches, random-init weights",
        "metric": "forecast series/sec",
        "value": round(rows / wall, 1),
        "unit": "series/s",
        "ms_per_call": round(wall * 1e3, 2),
        "device_forward_ms": round(dev_ms, 2),
        "device_series_per_s": round(rows / (dev_ms * 1e-3), 1),
        "gemm_tflops": round(gemm_flops / (dev_ms * 1e-3) / 1e12, 2),
    }
    del model
    torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=256)
    ap.add_argument("--only", choices=["all", "time", "group", "bf16", "fp16", "layer", "layer-bf16", "ts", "ts-block", "ts-block-bf16", "forecast"], default="all",
                    help="which workloads to run (profiling runs select one kernel)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run 5 plain device copies of this many bytes (calibrates rocprof byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (each series and each "
              "group is independent; see DESIGN.md for how the path would shard)", file=sys.stderr)
        return 2

    import torch

    import jitcast_amd
    from jitcast_amd import chronos2, synthetic

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_bytes:
        a = torch.empty(args.copy_bytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copied {args.copy_bytes} bytes 5 times")
        return 0
    also = {}
    if args.only in ("all", "forecast"):
        for name in ("bf16", "f32"):
            also[f"c2_forecast_{name}"] = forecast_line(2, 1, name)
        if args.only == "forecast":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "ts-block", "ts-block-bf16"):
        for name in (("bf16",) if args.only == "ts-block-bf16" else ("bf16", "f32")):
            also[f"ts_block_{name}"] = ts_block_line(2, 1, name)
        if args.only in ("ts-block", "ts-block-bf16"):
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "ts"):
        also["ts_time_attention_bf16"] = ts_time_attention_line(max(3, args.steps // 5), 1)
        if args.only == "ts":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "layer-bf16"):
        also["c2_layer_bf16"] = layer_line(max(3, args.steps // 5), 1, "bf16")
        if args.only == "layer-bf16":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "layer"):
        also["c2_layer_f32"] = layer_line(max(2, args.steps // 10), 1)
        if args.only == "layer":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "group") and args.only != "time":
        also["c2_group_attention_f32"] = group_attention_line(max(5, args.steps // 2), 2)
        if args.only == "group":
            print(json.dumps({"also": also}), flush=True)
            return 0
    log("generating config 1 inputs in HBM")
    case = synthetic.c2_time_config1(device="cuda")
    if args.only in ("all", "bf16", "fp16"):
        for name in (("bf16", "fp16") if args.only == "all" else (args.only,)):
            also[f"c2_time_attention_{name}"] = time_attention_lowp_line(case, args.steps, args.warmup, name)
        if args.only != "all":
            print(json.dumps({"also": also}), flush=True)
            return 0
    out = torch.empty(case.rows * case.n, case.inner, dtype=torch.float32, device=dev)
    flops = case.mask_aware_flops()
    dense = case.dense_flops()

    def step():
        chronos2.time_attention(case.qkv, out, case.live, case.rows, case.n, case.heads, case.dh, case.inner,
                                case.table)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} done; timing {args.steps} steps")
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in ev:
        a.record(stream)
        step()
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = sum(a.elapsed_time(b) for a, b in ev) / len(ev)
    ms_per_step = wall * 1e3 / args.steps
    value = flops / (ms_per_step * 1e-3) / 1e12
    achieved = flops / (launch_ms * 1e-3) / 1e12
    log(f"{ms_per_step:.4f} ms/step, kernel {launch_ms:.4f} ms, {achieved:.1f} TFLOP/s mask-aware, "
        f"{dense / (launch_ms * 1e-3) / 1e12:.1f} dense")

    cpu = None
    if not args.no_cpu_baseline:
        threads = os.cpu_count() or 1
        try:
            threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
        except ValueError:
            pass
        log(f"cpu baseline on {args.cpu_rows} rows with {threads} threads")
        cpu = cpu_baseline(case, args.cpu_rows, threads)

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (SplitMix64/Box-Muller seed 0: x~N(0,1), Wqkv~N(0,0.02), qkv=x Wqkv^T)",
        "config": {
            "workload": "config 1: isolated fp32 Chronos-2 time self-attention, RoPE at load, left padding "
                        "U{0..256} masked",
            "series": case.rows, "tokens": case.n, "heads": case.heads, "head_dim": case.dh,
            "d_model": case.inner, "flops_per_step_mask_aware": flops, "flops_per_step_dense": dense,
            "pct_of_fp32_mfma_peak": round(100 * value / PEAK_FP32_TFLOPS, 2),
            "dense_tflops": round(dense / (ms_per_step * 1e-3) / 1e12, 3),
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
            "traffic": traffic_from_profile("c2_time_attention_f32_config1"),
            "kernel": "jc::time_attention_f32<64, 32, true, false, true>",
            "launch_ms": round(launch_ms, 5),
        },
        "cpu_baseline": cpu,
        "also": also,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
