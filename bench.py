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


def traffic_source(name: str) -> str:
    """Where a roofline's traffic figure comes from: it is read from a committed profile, not measured
    in this run."""
    return (f"profiles/{name}.traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of the same kernel in "
            f"an earlier run, scaled by known-size copy, reduction and fill kernels (not measured in this run)")


def _profile(name: str) -> dict:
    p = ROOT / "profiles" / f"{name}.traffic.json"
    if not p.exists():
        return {}
    try:
        return json.loads(p.read_text())
    except Exception:
        return {}


def traffic_from_profile(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by
    known-size calibration kernels), committed as profiles/<name>.traffic.json; None when not
    measured."""
    return _profile(name).get("bytes_per_launch")


def from_profile(name: str, frac: float, launch_ms: float) -> dict:
    """The roofline fields read from a committed profile: the traffic, where it comes from, and the
    profiled box's own timing of the same kernel (20 launches after 5 warm-ups, as here) with the
    frac that timing gives and that box's clock from GRBM_GUI_ACTIVE. Boxes of the pool differ by
    several percent, so this frac and the live one bracket the box-to-box range."""
    d = _profile(name)
    out = {"traffic": d.get("bytes_per_launch"), "traffic_source": traffic_source(name)}
    ms = d.get("launch_ms")
    if ms:
        out["profiled_box"] = {"launch_ms": round(ms, 5), "frac": round(frac * launch_ms / ms, 4),
                               "clock_ghz": d.get("clock_ghz")}
    return out


def cpu_info(threads: int) -> dict:
    """The host CPU the baselines ran on: the model name (as lscpu reports it, from /proc/cpuinfo)
    and the threads used."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "threads": threads, "online_cpus": os.cpu_count()}


def cpu_threads() -> int:
    """The CPU share the baselines use: OMP_NUM_THREADS when set (the GPU box's per-GPU share),
    else every CPU."""
    threads = os.cpu_count() or 1
    try:
        threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    except ValueError:
        pass
    return max(1, threads)


def _oracle():
    sys.path.insert(0, str(ROOT))
    from oracle import oracle

    oracle.lib()
    return oracle


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
        **cpu_info(threads),
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


def group_attention_line(steps: int, warmup: int, cpu: bool = True) -> dict:
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
    # the same launches with fp32 storage on fp32 MFMA throughout instead of three-term fp16 products
    os.environ["JITCAST_HIP_GROUP_F32MMA"] = "1"
    try:
        ms32 = time_launches(fn, steps, warmup)
    finally:
        del os.environ["JITCAST_HIP_GROUP_F32MMA"]
    log(f"group attention on fp32 MFMA: {ms32:.4f} ms ({100 * nbytes / (ms32 * 1e-3) / 1e9 / PEAK_HBM_GBS:.1f}% of HBM)")
    res = {
        "workload": "config 2: fp32 Chronos-2 group attention, 4096 rows x 129 slots, 12x64, groups U{1..64}",
        "kernel": "jc::group_attention_f32<float, 64, false, true, false>",
        "launch_ms": round(ms, 5),
        "value": round(gbs, 1),
        "unit": "GB/s",
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), **from_profile("c2_group_attention_f32_config2", gbs / PEAK_HBM_GBS, ms)},
        "bytes_per_launch": nbytes,
        "tflops": round(case.flops() / (ms * 1e-3) / 1e12, 2),
        "products": "three-term fp16 MFMA products (v = hi + lo), fp32 softmax and accumulation",
        "fp32_mfma_launch_ms": round(ms32, 5),
    }
    if cpu:
        res["cpu_baseline"] = group_cpu_baseline(case, cpu_threads())
    del case, out
    torch.cuda.empty_cache()
    return res


def group_cpu_baseline(case, threads: int, sample_rows: int = 4096) -> dict:
    """The oracle's CpuChronos2.groupAttention on the first whole groups of config 2 (about
    sample_rows rows), in the GPU figure's unit: algorithmic bytes of the sample per second."""
    import numpy as np

    oracle = _oracle()
    ends = np.flatnonzero(np.diff(case.group)) + 1
    rows = int(ends[ends <= sample_rows].max()) if (ends <= sample_rows).any() else case.rows
    n, inner = case.n, case.inner
    qkv = case.qkv[: rows * n].cpu().numpy()
    live = case.live[: rows * n].cpu().numpy().astype(np.int32)
    t0 = time.perf_counter()
    oracle.c2_group_attention(qkv, live, case.group[:rows], rows, n, case.heads, case.dh, inner, threads=threads)
    dt = time.perf_counter() - t0
    nbytes = float(rows) * n * 4 * inner * 4
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the first {rows} of {case.rows} rows (whole groups) of config 2, {dt:.2f} s, double accumulation",
            **cpu_info(threads)}


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
                     **from_profile(f"c2_time_attention_{dtype_name}_config1", tf / PEAK_BF16_TFLOPS, ms)},
        "dense_tflops": round(case.dense_flops() / (ms * 1e-3) / 1e12, 2),
    }
    del q16, out
    torch.cuda.empty_cache()
    return res


def layer_line(steps: int, warmup: int, dtype_name: str = "f32") -> dict:
    """Config 4's encoder-layer shape through jc_c2_layer: RMSNorm, the six GEMMs of the layer, RoPE
    time attention, group attention, ReLU and the residual adds. f32: everything fp32. bf16: the
    GEMMs and the time attention in bf16 with fp32 accumulation (weights converted once, outside the
    timed region), the group attention, norms and residual stream fp32. f16x3: f32's layer with every
    GEMM on three-term fp16 splits of its operands (weights split once, outside the timed region)."""
    import torch

    from jitcast_amd import _lib, chronos2, synthetic

    case = synthetic.c2_layer_config4(device="cuda")
    code = {"f32": _lib.JC_F32, "bf16": _lib.JC_BF16, "f16x3": _lib.JC_F16X3}[dtype_name]
    weights = dict(case.weights)
    ws = case.workspace
    if code == _lib.JC_F16X3:
        for k in ("time_qkv", "time_o", "group_qkv", "group_o", "wi", "wo"):
            x3 = torch.empty(weights[k].shape[0], 3 * weights[k].shape[1], dtype=torch.float16, device="cuda")
            chronos2.split_f16x3(weights[k].contiguous(), x3, weights=True)
            weights[k] = x3
        inner = case.heads * case.dh
        ws = torch.empty(chronos2.layer_workspace_bytes(case.rows, case.n, case.d, inner, case.dff, code) // 4 + 64,
                         dtype=torch.float32, device="cuda")
    elif code != _lib.JC_F32:
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
    # f16x3 runs its GEMMs on fp16 MFMA, three products per fp32 product: it is priced against the fp16
    # peak with the algorithmic (fp32) flops, and the executed MFMA flops are reported beside them
    peak = PEAK_FP32_TFLOPS if code == _lib.JC_F32 else PEAK_BF16_TFLOPS
    tokens = case.rows * case.n
    peak_name = {"f16x3": "fp16 MFMA peak, fp32-equivalent flops"}.get(dtype_name, f"{dtype_name} MFMA peak")
    log(f"layer {dtype_name}: {ms:.3f} ms, {tf:.1f} TFLOP/s ({100 * tf / peak:.1f}% of the {peak_name}), "
        f"{tokens / (ms * 1e-3) / 1e6:.1f} M tokens/s")
    res = {
        "workload": f"config 4 encoder-layer shape: 1024 groups x (4 series + 1 known covariate), 133 tokens "
                    f"(128 context patches + REG + 4 future), d_model 768, 12x64, d_ff 3072, {dtype_name}",
        "kernel": "jc_c2_layer (hipBLASLt %s GEMMs)" % {_lib.JC_F32: "fp32", _lib.JC_BF16: "bf16 x bf16 -> fp32 / bf16",
                                                         _lib.JC_F16X3: "fp16 (three-term splits, K = 3k)"}[code],
        "launch_ms": round(ms, 4),
        "value": round(tf, 2),
        "unit": "TFLOP/s",
        "tokens_per_s": round(tokens / (ms * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tf / peak, 4),
                     **from_profile(f"c2_layer_{dtype_name}_config4", tf / peak, ms)},
        "flops_per_step": flops,
        "gemm_share_of_flops": round(case.gemm_flops() / flops, 4),
    }
    if code == _lib.JC_F16X3:
        res["executed_tflops"] = round((flops + 2 * case.gemm_flops()) / (ms * 1e-3) / 1e12, 2)
    del case, x0, weights, ws
    torch.cuda.empty_cache()
    return res


def ts_time_attention_line(steps: int, warmup: int, cpu: bool = True) -> dict:
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
    log(f"config 3 attention bf16: {ms:.3f} ms for {layers} launches, {tf:.1f} TFLOP/s mask-aware "
        f"({100 * tf / PEAK_BF16_TFLOPS:.1f}% of the bf16 MFMA peak)")
    res = {
        "workload": "config 3: Timestral time attention in bf16 (RoPE on half the head, bidirectional over valid "
                    "keys, left padding U{0..256}, fused gate), 64 series x 1024 tokens, 12x64, 12 launches per step",
        "kernel": "jc::time_attention_lp<__bf16, 64, 4, true, true, true>",
        "launch_ms": round(ms / layers, 5),
        "value": round(tf, 2),
        "unit": "TFLOP/s",
        "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                     **from_profile("ts_time_attention_bf16_config3", tf / PEAK_BF16_TFLOPS, ms / layers)},
        "dense_tflops": round(layers * 4.0 * case.dh * case.n * case.n * case.heads * case.rows / (ms * 1e-3) / 1e12, 2),
    }
    res["stack"] = ts_stack_timing(case, steps, warmup)
    if cpu:
        res["cpu_baseline"] = ts_time_cpu_baseline(case, cpu_threads())
    del case, out
    torch.cuda.empty_cache()
    return res


def ts_stack_timing(case, steps: int, warmup: int) -> dict:
    """Config 3's whole attention stack through HipTimestralModel.encoder: 12 layers of RMSNorm,
    q|k|v and gate projections, the fused time attention and the output projection added to x, in
    bf16 with fp32 accumulation (N(0, 0.02) weights, x ~ N(0, 1)); TFLOP/s over its GEMMs and
    mask-aware attention flops."""
    import torch

    from jitcast_amd import rng
    from jitcast_amd import timestral_model as tm
    from jitcast_amd.runtime import fill_normal

    c = tm.TimestralConfig(layers=((True,),) * 12)
    model = tm.HipTimestralModel(c, tm.random_weights(c, seed=0), dtype="bf16")
    rows, n, d = case.rows, case.n, case.d
    x0 = torch.empty(rows * n, d, dtype=torch.float32, device=model.dev)
    fill_normal(x0, rng.stream_seed(0, 23), 0.0, 1.0)
    x = x0.clone()
    known = torch.ones(rows, dtype=torch.int32, device=model.dev)

    def fn():
        model.encoder(x, case.key_valid, known, case.pos, None, None, None, False, rows, n, 0, mlp=False)

    ms = time_launches(fn, max(2, steps // 2), 1)
    gemm = 2.0 * rows * n * len(c.layers) * 5 * d * d
    attn = len(c.layers) * case.mask_aware_flops()
    tf = (gemm + attn) / (ms * 1e-3) / 1e12
    log(f"config 3 attention stack bf16 (12 layers with projections): {ms:.3f} ms, {tf:.1f} TFLOP/s "
        f"({100 * tf / PEAK_BF16_TFLOPS:.1f}% of the bf16 MFMA peak), {rows / (ms * 1e-3):.0f} series/s")
    del model, x, x0
    torch.cuda.empty_cache()
    return {"ms": round(ms, 4), "tflops": round(tf, 2), "frac": round(tf / PEAK_BF16_TFLOPS, 4),
            "series_per_s": round(rows / (ms * 1e-3), 1), "gemm_flops": gemm, "attention_flops": attn}


def ts_time_cpu_baseline(case, threads: int, sample_rows: int = 64) -> dict:
    """The oracle's CpuTimestral.timeAttention on sample_rows series of config 3's shape (fp32, the
    bf16 inputs widened), mask-aware TFLOP/s."""
    import numpy as np

    oracle = _oracle()
    rows, n, d = sample_rows, case.n, case.d
    qkv = case.qkv[: rows * n].float().cpu().numpy()
    kv = case.key_valid[: rows * n].cpu().numpy().astype(np.int32)
    known = np.ones(rows, np.int32)
    pos = case.pos[: rows * n].cpu().numpy().astype(np.int32) - n
    t0 = time.perf_counter()
    oracle.ts_time_attention(qkv, kv, known, pos, rows, n, n, n, case.heads, case.dh, d, 32, threads=threads)
    dt = time.perf_counter() - t0
    per_row = [(n - s) * n + s for s in case.starts[:rows]]
    flops = 4.0 * case.dh * case.heads * float(sum(per_row))
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of {case.rows} series of config 3 (1024 tokens, 12x64), mask-aware flops, {dt:.2f} s, "
                      "double accumulation", **cpu_info(threads)}


def chronos2_bench_timing(call, warmup: int = 3, reps: int = 20, budget_s: float = 5.0) -> dict:
    """Chronos2Bench's method (J/bench/Chronos2Bench.java:63-84): a first run, `warmup` more, then
    up to `reps` timed runs within a budget of `budget_s` seconds (at least 3); the median and min."""
    import torch

    t0 = time.perf_counter()
    call()
    torch.cuda.synchronize()
    first = (time.perf_counter() - t0) * 1e3
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    ms = []
    deadline = time.perf_counter() + budget_s
    while len(ms) < reps and (len(ms) < 3 or time.perf_counter() < deadline):
        t0 = time.perf_counter()
        call()
        torch.cuda.synchronize()
        ms.append((time.perf_counter() - t0) * 1e3)
    ms.sort()
    k = len(ms)
    median = ms[k // 2] if k % 2 else (ms[k // 2 - 1] + ms[k // 2]) / 2
    return {"median_ms": round(median, 3), "min_ms": round(ms[0], 3), "first_ms": round(first, 3), "reps": k}


def c4_series():
    """Config 4's request as ForecastEngine input: 1024 TimeSeries, each 4 target rows of 2048 steps
    and one known-future covariate of 2048 + 64 steps (synthetic.c2_forecast_config4's values)."""
    import numpy as np

    from jitcast_amd.api import TimeSeries
    from jitcast_amd import synthetic

    ctx, group, fut, targets = synthetic.c2_forecast_config4()
    series = []
    for g in range(1024):
        rows = np.flatnonzero(group == g)
        tg = rows[targets[rows]]
        cov = rows[~targets[rows]]
        known = np.concatenate([ctx[cov], fut[cov]], axis=1)
        series.append(TimeSeries(ctx[tg], None, known))
    return series, int(targets.sum())


def forecast_line(ckpt_dir, series, n_targets: int, dtype_name: str = "f32", cpu: bool = False) -> dict:
    """Config 4 end to end through the engine: HipChronos2Engine.load(config.json + model.safetensors of
    the 120M-class random-init model), then ForecastEngine.forecast of 1024 series (4 targets + 1
    known-future covariate, 2048 steps) at horizon 64, 21 quantiles: the pipeline's ≤256-row batches
    make 20 forward calls (19 x 260 rows, 1 x 180). value = TimeSeries forecast per second (1024 / the
    median forecast() wall time, Chronos2Bench's method, J/bench/Chronos2Bench.java:63-84), with
    target rows per second (4096 / t) beside it. Also: the same forecast with each call's device
    forward replayed from its plan (one hipGraph per batch shape), a 20-row request eager and from the
    plan, and the device forward of one 260-row call alone (HIP events). The first forecast, the same
    request after every timed run and the first forecast from plans must agree bit for bit."""
    import numpy as np
    import torch

    from jitcast_amd import chronos2_model as cm
    from jitcast_amd.engine import HipChronos2Engine

    h = 64
    calls = []
    with HipChronos2Engine.load(ckpt_dir, dtype=dtype_name, max_plans=0) as eng:
        fwd = eng.pipeline().forward
        eng.pipeline().forward = lambda inp: calls.append(inp.rows()) or fwd(inp)
        out = eng.forecast(series, h)
        eng.pipeline().forward = fwd
        t = chronos2_bench_timing(lambda: eng.forecast(series, h))
        small = series[:4]
        lat_eager = chronos2_bench_timing(lambda: eng.forecast(small, h), budget_s=1.0)
        # one 260-row call's device forward alone
        c = eng.config()
        rows = 260
        ctx = np.stack([r for s in series[:52] for r in list(s.target) + [s.future_covariates[0][:2048]]])
        group = np.repeat(np.arange(52, dtype=np.int32), 5)
        lay = cm.layout(c, ctx, group, None, h // c.patch_size)
        tok, _, _ = cm.prep(c, lay)
        gs, ge = cm.chronos2.group_bounds(lay.group)
        model = eng.forward_pass().model
        dev = model.dev
        args = (torch.from_numpy(tok).to(dev), torch.from_numpy(lay.live.reshape(-1)).to(dev),
                torch.from_numpy(gs).to(dev), torch.from_numpy(ge).to(dev), rows, lay.nc, lay.h)
        dev_ms = time_launches(lambda: model.forward_raw(*args), 5, 1)
        again = eng.forecast(series, h)  # the first request again, after every timed run
    with HipChronos2Engine.load(ckpt_dir, dtype=dtype_name, max_plans=4) as peng:
        pout = peng.forecast(series, h)
        tp = chronos2_bench_timing(lambda: peng.forecast(series, h))
        lat_plan = chronos2_bench_timing(lambda: peng.forecast(series[:4], h), budget_s=1.0)
        pagain = peng.forecast(series, h)  # from the cached plans, after every timed run
    assert all(np.isfinite(f.values).all() for f in out) and all(np.isfinite(f.values).all() for f in pout)
    # a plan replays the eager task graph (Chronos2Forward.java:292-300) and the same request gives the
    # same forecast: both must hold bit for bit, or the run fails
    scale = max(float(np.max(np.abs(a.values))) for a in out)
    repro = {}
    for name, other in (("eager_vs_eager", again), ("plan_vs_eager", pout), ("plan_again_vs_eager", pagain)):
        n_diff = sum(not np.array_equal(a.values, b.values) for a, b in zip(out, other))
        max_diff = max(float(np.max(np.abs(a.values - b.values))) for a, b in zip(out, other))
        repro[name] = {"series_differing": n_diff, "max_abs_diff": max_diff}
        if n_diff:
            raise AssertionError(f"forecast {dtype_name}: {name.replace('_', ' ')} differs in {n_diff} of {len(out)} "
                                 f"series (max abs diff {max_diff:.3e}, forecast scale {scale:.3e})")
    n_series = len(series)
    sps = n_series / (t["median_ms"] * 1e-3)
    rps = n_targets / (t["median_ms"] * 1e-3)
    log(f"forecast {dtype_name} through the engine: median {t['median_ms']:.1f} ms per forecast() of {n_series} series "
        f"({len(calls)} forward calls of {calls[0]}..{calls[-1]} rows), {sps:.1f} series/s ({rps:.0f} target rows/s); "
        f"from plans {tp['median_ms']:.1f} ms; one 260-row device forward {dev_ms:.2f} ms; 4-series request "
        f"{lat_eager['median_ms']:.2f} ms eager, {lat_plan['median_ms']:.2f} ms from its plan; eager and plan "
        f"forecasts bit-identical")
    encoder = {"f32": "fp32 encoder, inside the 1e-3 quantile bar",
               "f16x3": "f16x3 encoder: fp32 GEMM results from three fp16 products each, inside the 1e-3 bar for "
                        "these inputs; its operands saturate at +-65504 (fp16's range), unlike fp32",
               "bf16": "bf16 encoder GEMMs and time attention (fp32 accumulation), the 2e-2 bar"}.get(dtype_name, dtype_name)
    res = {
        "workload": f"config 4: Chronos-2 120M-class forecast() through HipChronos2Engine ({encoder}), "
                    f"{n_series} series x (4 targets + 1 known-future covariate) x 2048 steps, horizon 64, 21 "
                    "quantiles, random-init weights loaded from config.json + model.safetensors",
        "metric": "forecast series/sec",
        "value": round(sps, 2),
        "unit": "series/s (TimeSeries of 4 targets + 1 covariate)",
        "target_rows_per_s": round(rps, 1),
        "timing": t,
        "forward_calls": len(calls), "rows_per_call": [calls[0], calls[-1]],
        "plan_timing": tp, "plan_series_per_s": round(n_series / (tp["median_ms"] * 1e-3), 2),
        "small_request": {"series": 4, "rows": 20, "eager": lat_eager, "plan": lat_plan},
        "device_forward_260_rows_ms": round(dev_ms, 3),
        "reproducible": {**repro, "forecast_scale": scale},
    }
    if cpu:
        res["cpu_baseline"] = forecast_cpu_baseline(ckpt_dir, series, cpu_threads())
    return res


def ts_forecast_line(dtype_name: str = "f32", rows: int = 64, steps: int = 16384, horizon: int = 64) -> dict:
    """The Timestral engine end to end: HipTimestralEngine.load(config.json + model.safetensors of the
    123M-class random-init model, the shape of config 3's stack with its MLPs and head), then
    ForecastEngine.forecast of `rows` univariate series of `steps` steps (config 0's sines + trend +
    noise; 16,384 steps are config 3's 1,024 patch tokens) at `horizon`, sign-flip averaging on (two
    block calls). value = series forecast per second from the median forecast() wall time
    (Chronos2Bench's method), from plans (the default) and eagerly; both must agree bit for bit."""
    import shutil
    import tempfile

    import numpy as np

    from jitcast_amd import checkpoint, synthetic
    from jitcast_amd import timestral_model as tm
    from jitcast_amd.api import TimeSeries
    from jitcast_amd.engine import HipTimestralEngine

    c = tm.TimestralConfig()
    x = synthetic.c2_config0_series(rows, steps, seed=3)
    series = [TimeSeries.univariate(r) for r in x]
    ckpt = Path(tempfile.mkdtemp(prefix="ts_engine_"))
    try:
        log(f"writing the Timestral 123M-class random-init checkpoint ({dtype_name} engine)")
        checkpoint.write_timestral(ckpt, c, tm.random_weights(c, seed=0, std=0.02))
        res = {}
        for plans in (8, 0):
            with HipTimestralEngine.load(ckpt, dtype=dtype_name, max_plans=plans) as eng:
                calls = []
                fwd = eng.pipeline().forward
                eng.pipeline().forward = lambda inp, *a: calls.append(np.shape(inp)) or fwd(inp, *a)
                out = eng.forecast(series, horizon)
                eng.pipeline().forward = fwd
                res[plans] = (out, chronos2_bench_timing(lambda: eng.forecast(series, horizon), budget_s=4.0), calls)
    finally:
        shutil.rmtree(ckpt, ignore_errors=True)
    (out, t, calls), (eout, te, _) = res[8], res[0]
    assert all(np.array_equal(a.values, b.values) for a, b in zip(out, eout)), "plan replay differs from eager"
    assert all(np.isfinite(f.values).all() for f in out)
    sps = rows / (t["median_ms"] * 1e-3)
    log(f"timestral forecast {dtype_name} through the engine: median {t['median_ms']:.1f} ms per forecast() of "
        f"{rows} series ({len(calls)} block calls of {calls[0]}), {sps:.0f} series/s; eager "
        f"{te['median_ms']:.1f} ms")
    return {
        "workload": f"Timestral 123M-class forecast() through HipTimestralEngine ({dtype_name}), {rows} univariate "
                    f"series x {steps} steps, horizon {horizon}, 9 quantiles, sign-flip averaging, random-init "
                    "weights loaded from config.json + model.safetensors",
        "metric": "forecast series/sec",
        "value": round(sps, 1),
        "unit": "series/s",
        "timing": t,
        "block_calls": len(calls), "block_shape": list(calls[0]),
        "eager_timing": te, "eager_series_per_s": round(rows / (te["median_ms"] * 1e-3), 1),
    }


def forecast_cpu_baseline(ckpt_dir, series, threads: int, groups: int = 4) -> dict:
    """The oracle (CpuChronos2.forward under ModelLayout, ModelPrep and finish) on one forward call of
    `groups` config-4 series (5 rows each), scaled linearly to target series per second: without
    cross-learning the work is linear in series. Labelled as extrapolated."""
    import numpy as np

    from jitcast_amd import checkpoint as ck

    oracle = _oracle()
    c, w = ck.load_chronos2(ckpt_dir)
    ctx = np.stack([r for s in series[:groups] for r in list(s.target) + [s.future_covariates[0][:2048]]])
    fut = np.full((ctx.shape[0], 64), np.nan, np.float32)
    fut[4::5] = np.stack([s.future_covariates[0][2048:2048 + 64] for s in series[:groups]])
    group = np.repeat(np.arange(groups, dtype=np.int32), 5)
    t0 = time.perf_counter()
    oracle.c2_model_forward(c, w, ctx, group, fut, 4, threads=threads)
    dt = time.perf_counter() - t0
    return {"value": round(4 * groups / dt, 4), "unit": "target series/s", "cores": threads, "kind": "port",
            "sample": f"one forward call of {groups} of the 1024 series ({5 * groups} rows x 133 tokens), {dt:.1f} s, "
                      "scaled linearly to series/s (extrapolated)", **cpu_info(threads)}


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
        "traffic_per_device_forward": traffic_from_profile(f"ts_block_{dtype_name}_config3"), "traffic_source": traffic_source(f"ts_block_{dtype_name}_config3"),
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
    ap.add_argument("--only", choices=["all", "time", "group", "bf16", "fp16", "layer", "layer-bf16", "layer-f16x3", "ts", "ts-block", "ts-block-bf16", "ts-forecast", "forecast"], default="all",
                    help="which workloads to run (profiling runs select one kernel)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run 5 plain device copies of this many bytes (calibrates rocprof byte counters)")
    ap.add_argument("--read-bytes", type=int, default=0,
                    help="only run 5 sums over this many bytes of fp32 (a read stream: calibrates FETCH_SIZE)")
    ap.add_argument("--write-bytes", type=int, default=0,
                    help="only run 5 fills of this many bytes of fp32 (a write stream: calibrates WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (each series and each "
              "group is independent, so the path would shard by whole groups of rows, one share per GPU)",
              file=sys.stderr)
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
    if args.read_bytes:
        a = torch.empty(args.read_bytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
        torch.cuda.synchronize()
        total = [a.sum() for _ in range(5)]
        torch.cuda.synchronize()
        log(f"summed {args.read_bytes} bytes 5 times ({float(total[-1]):.0f})")
        return 0
    if args.write_bytes:
        a = torch.empty(args.write_bytes // 4, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        for v in range(5):
            a.fill_(float(v))
        torch.cuda.synchronize()
        log(f"filled {args.write_bytes} bytes 5 times")
        return 0
    also = {}
    want_cpu = not args.no_cpu_baseline
    if args.only in ("all", "forecast"):
        import shutil
        import tempfile

        from jitcast_amd import checkpoint, synthetic
        from jitcast_amd.chronos2_model import Chronos2Config

        c4 = Chronos2Config()  # 120M-class: d_model 768, 12 x 64, 12 layers, d_ff 3072, patch 16, 21 quantiles
        ckpt = Path(tempfile.mkdtemp(prefix="c2_config4_"))
        try:
            log("writing config 4's random-init checkpoint (config.json + model.safetensors)")
            checkpoint.write_chronos2(ckpt, c4, synthetic.c2_portable_weights(c4, seed=0))
            series, n_targets = c4_series()
            # fp32 first: the encoder inside config 4's 1e-3 quantile bar
            also["c2_forecast_f32"] = forecast_line(ckpt, series, n_targets, "f32")
            # f16x3: fp16 GEMMs over three-term splits, inside the same 1e-3 bar
            also["c2_forecast_f16x3"] = forecast_line(ckpt, series, n_targets, "f16x3")
            also["c2_forecast_bf16"] = forecast_line(ckpt, series, n_targets, "bf16")
            if want_cpu:  # the oracle's forward, after the device forecasts
                also["c2_forecast_f32"]["cpu_baseline"] = forecast_cpu_baseline(ckpt, series, cpu_threads())
        finally:
            shutil.rmtree(ckpt, ignore_errors=True)
        if args.only == "forecast":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only == "ts-forecast":  # the Timestral host pipeline: outside the attention path, not in the default run
        for name in ("bf16", "f16x3", "f32"):
            also[f"ts_forecast_{name}"] = ts_forecast_line(name)
        if args.only == "ts-forecast":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "ts-block", "ts-block-bf16"):
        for name in (("bf16",) if args.only == "ts-block-bf16" else ("bf16", "f16x3", "f32")):
            also[f"ts_block_{name}"] = ts_block_line(2, 1, name)
        if args.only in ("ts-block", "ts-block-bf16"):
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "ts"):
        also["ts_time_attention_bf16"] = ts_time_attention_line(max(3, args.steps // 5), 1, cpu=want_cpu)
        if args.only == "ts":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "layer-bf16", "layer-f16x3"):
        for name in (("bf16", "f16x3") if args.only == "all" else (args.only[6:],)):
            also[f"c2_layer_{name}"] = layer_line(max(3, args.steps // 5), 1, name)
        if args.only != "all":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "layer"):
        also["c2_layer_f32"] = layer_line(max(2, args.steps // 10), 1)
        if args.only == "layer":
            print(json.dumps({"also": also}), flush=True)
            return 0
    if args.only in ("all", "group") and args.only != "time":
        also["c2_group_attention_f32"] = group_attention_line(max(5, args.steps // 2), 2, cpu=want_cpu)
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
    if want_cpu:
        threads = cpu_threads()
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
            **from_profile("c2_time_attention_f32_config1", achieved / PEAK_FP32_TFLOPS, launch_ms),
            "kernel": "jc::time_attention_f32<64, 32, true, false, true, true, false>",
            "launch_ms": round(launch_ms, 5),
        },
        "cpu_baseline": cpu,
        "also": also,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
