"""The HIP Chronos-2 engine: ForecastEngine over the shared host pipeline and the device forward, as
TornadoChronos2Engine is over Chronos2Forward (J/chronos2/tornado/TornadoChronos2Engine.java:30-111).

  HipChronos2Forward  ModelForward.forward (J/chronos2/ModelForward.java:20-23) on the GPU: one
                      HipChronos2Model.forecast per call (the group order, ModelLayout and ModelPrep,
                      the encoder, finish), eager or replayed from a plan per batch shape
  HipChronos2Engine   load(checkpoint_dir) / forecast(series, horizon) / name() / close(); config(),
                      forward_pass() and pipeline() as the reference's engine exposes them
  HipTimestralEngine  the same over TimestralPipeline (ts_pipeline.py) and HipTimestralModel.predict_block,
                      as TornadoTimestralEngine (J/timestral/tornado/TornadoTimestralEngine.java:29-111)

Settings come from the arguments or, when an argument is None, from the -D properties (options.py):
chronos2.hip.dtype, chronos2.hip.plans, chronos2.hip.planBytes, timestral.hip.dtype,
timestral.hip.plans, timestral.hip.planBytes, timestral.hip.buckets, jitcast.hip.device.
"""
from __future__ import annotations

import threading

import numpy as np

from . import options as opts
from .api import ForecastEngine
from .pipeline import Chronos2Pipeline, ModelInput


class HipChronos2Forward:
    """The device forward pass under the pipeline: ModelInput -> float32 [rows, Q, output_patches*P]."""

    def __init__(self, config, weights: dict, dtype: str = "f32", device: int = 0, max_plans: int = 0,
                 plan_bytes: int | None = None):
        from .chronos2_model import HipChronos2Model

        self.config = config
        self.model = HipChronos2Model(config, weights, dtype=dtype, device=device, max_plans=max_plans,
                                      plan_bytes=plan_bytes)

    def __call__(self, inp: ModelInput) -> np.ndarray:
        return self.forward(inp)

    def forward(self, inp: ModelInput) -> np.ndarray:
        return self.model.forecast(inp.context, inp.group, inp.future_covariates, h=inp.output_patches)

    def close(self) -> None:
        self.model.close()


class HipChronos2Engine(ForecastEngine):
    """Chronos-2 on one GPU. The engine owns its weights (uploaded once) and releases them in close().
    Calls from several threads run one at a time, since they share the device buffers."""

    def __init__(self, config, weights: dict, dtype: str | None = None, device: int | None = None,
                 max_plans: int | None = None, plan_bytes: int | None = None, pipeline_options=None,
                 batch_size: int | None = None, max_tokens: int | None = None):
        dtype = dtype if dtype is not None else opts.choice("chronos2.hip.dtype", "f32", "f32", "bf16", "fp16", "f16x3")
        if dtype not in ("f32", "bf16", "fp16", "f16x3"):
            raise ValueError(f"dtype must be f32, bf16, fp16 or f16x3, got {dtype}")
        device = device if device is not None else opts.integer("jitcast.hip.device", 0, 0)
        max_plans = max_plans if max_plans is not None else opts.integer("chronos2.hip.plans", 8, 0)
        if plan_bytes is None and max_plans > 0:
            import torch

            total = torch.cuda.get_device_properties(device).total_memory
            plan_bytes = opts.bytes_("chronos2.hip.planBytes", total, 1)
        self._config = config
        self._dtype = dtype
        self._forward = HipChronos2Forward(config, weights, dtype=dtype, device=device, max_plans=max_plans,
                                           plan_bytes=plan_bytes)
        kw = {}
        if batch_size is not None:
            kw["batch_size"] = batch_size
        self._pipeline = Chronos2Pipeline(config, self._forward, pipeline_options, max_tokens=max_tokens, **kw)
        self._lock = threading.Lock()
        self._closed = False

    @staticmethod
    def load(checkpoint_dir, **kw) -> "HipChronos2Engine":
        """An engine over <dir>/config.json and <dir>/model.safetensors (TornadoChronos2Engine.load);
        the load fails on unknown config keys, unsupported settings and missing, misshapen or extra
        tensors."""
        from .checkpoint import load_chronos2

        config, weights = load_chronos2(checkpoint_dir)
        return HipChronos2Engine(config, weights, **kw)

    def config(self):
        return self._config

    def forward_pass(self) -> HipChronos2Forward:
        """The device forward pass under the pipeline, for benchmarks and tests."""
        return self._forward

    def pipeline(self) -> Chronos2Pipeline:
        """The host pipeline forecast() runs; its with_* methods give pipelines with other settings over
        this engine's forward pass."""
        return self._pipeline

    def forecast(self, series: list, horizon: int) -> list:
        with self._lock:
            if self._closed:
                raise RuntimeError("the engine is closed")
            return self._pipeline.forecast(series, horizon)

    def name(self) -> str:
        return "chronos2-hip" if self._dtype == "f32" else f"chronos2-hip-{self._dtype}"

    def close(self) -> None:
        with self._lock:
            if self._closed:
                return
            self._closed = True
            self._forward.close()
            self._forward.model = None


class HipTimestralEngine(ForecastEngine):
    """Timestral on one GPU: TimestralPipeline around HipTimestralModel.predict_block. The engine owns its
    weights (uploaded once) and releases them in close(); calls from several threads run one at a time."""

    def __init__(self, config, weights: dict, dtype: str | None = None, device: int | None = None,
                 max_plans: int | None = None, plan_bytes: int | None = None, buckets: bool | None = None,
                 pipeline_options=None, batch_size: int | None = None, max_tokens: int | None = None):
        from .timestral_model import HipTimestralModel
        from .ts_pipeline import DEFAULT_BATCH_SIZE, TimestralPipeline

        dtype = dtype if dtype is not None else opts.choice("timestral.hip.dtype", "f32", "f32", "bf16", "fp16", "f16x3")
        if dtype not in ("f32", "bf16", "fp16", "f16x3"):
            raise ValueError(f"dtype must be f32, bf16, fp16 or f16x3, got {dtype}")
        device = device if device is not None else opts.integer("jitcast.hip.device", 0, 0)
        self._config = config
        self._dtype = dtype
        self._model = HipTimestralModel(config, weights, dtype=dtype, device=device, max_plans=max_plans,
                                        plan_bytes=plan_bytes, buckets=buckets)
        self._pipeline = TimestralPipeline(config, self._model.predict_block, pipeline_options,
                                           batch_size if batch_size is not None else DEFAULT_BATCH_SIZE, max_tokens)
        self._lock = threading.Lock()
        self._closed = False

    @staticmethod
    def load(checkpoint_dir, **kw) -> "HipTimestralEngine":
        """An engine over <dir>/config.json and <dir>/model.safetensors (TornadoTimestralEngine.load); the
        load fails on unknown config keys, unsupported settings and missing, misshapen or extra tensors."""
        from .checkpoint import load_timestral

        config, weights = load_timestral(checkpoint_dir)
        return HipTimestralEngine(config, weights, **kw)

    def config(self):
        return self._config

    def forward_pass(self):
        """The device block forward under the pipeline (HipTimestralModel), for benchmarks and tests."""
        return self._model

    def pipeline(self):
        """The host pipeline forecast() runs; its with_* methods give pipelines with other settings over
        this engine's forward pass."""
        return self._pipeline

    def forecast(self, series: list, horizon: int) -> list:
        with self._lock:
            if self._closed:
                raise RuntimeError("the engine is closed")
            return self._pipeline.forecast(series, horizon)

    def name(self) -> str:
        return "timestral-hip" if self._dtype == "f32" else f"timestral-hip-{self._dtype}"

    def close(self) -> None:
        with self._lock:
            if self._closed:
                return
            self._closed = True
            self._model.close()
