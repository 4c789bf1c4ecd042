"""Chronos-2's host pipeline: series in, quantile forecasts out, over any forward pass
(J/chronos2/Chronos2Pipeline.java:43-464).

  ModelInput        one forward call's arguments (J/chronos2/ModelInput.java:28): context
                    [rows, T] (NaN where missing), group [rows], future covariates
                    [rows, output_patches * P] (NaN where unknown), output_patches
  Options           context cap, cross-learning, patches per pass, the unrolled levels
                    (Chronos2Pipeline.Options, Chronos2Pipeline.java:60-90)
  Chronos2Pipeline  forecast(series, horizon): each series' rows (targets, past covariates, known
                    covariates), batches of at most batch_size rows, NaN left-padding, one group
                    per series (or one per batch with cross-learning), the long-horizon unrolling
                    and the token-budget split into passes of whole groups

A forward pass is any callable ModelInput -> float32 [rows, Q, output_patches * P] in each row's
own scale (ModelForward.forward, J/chronos2/ModelForward.java:20-23): the HIP engine's, or the
oracle's in the tests.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable

import numpy as np

from . import options as opts
from . import quantile_math as qm
from .api import Forecast, TimeSeries

F32 = np.float32
DEFAULT_BATCH_SIZE = 256
UNROLLED = (0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8, 0.9)


def default_max_tokens() -> int:
    """-Dchronos2.maxTokens, default 131,072 (Chronos2Pipeline.defaultMaxTokens)."""
    return opts.number("chronos2.maxTokens", 131_072, 1)


@dataclass(frozen=True)
class ModelInput:
    context: np.ndarray  # float32 [rows, T]
    group: np.ndarray  # int32 [rows]
    future_covariates: np.ndarray  # float32 [rows, output_patches * P]
    output_patches: int

    def rows(self) -> int:
        return int(self.context.shape[0])

    def length(self) -> int:
        return int(self.context.shape[1])


@dataclass(frozen=True)
class Options:
    context_length: int
    cross_learning: bool
    max_output_patches: int
    unrolled_quantiles: tuple = field(default=UNROLLED)

    @staticmethod
    def defaults(c) -> "Options":
        """The reference's settings for a checkpoint: its context cap, no cross-learning, its
        patches per pass, levels 0.1..0.9 fed back."""
        return Options(c.context_length, False, c.max_output_patches, UNROLLED)

    def with_cross_learning(self, on: bool) -> "Options":
        return Options(self.context_length, bool(on), self.max_output_patches, self.unrolled_quantiles)

    def with_context_length(self, steps: int) -> "Options":
        return Options(int(steps), self.cross_learning, self.max_output_patches, self.unrolled_quantiles)


@dataclass
class _Prepared:
    context: list  # float32 rows, each min(T, cap) steps
    future: np.ndarray  # float32 [rows, horizon]
    targets: int


class Chronos2Pipeline:
    """Chronos2Pipeline over a forward pass `forward` (ModelInput -> [rows, Q, steps])."""

    def __init__(self, config, forward: Callable, options: Options | None = None, batch_size: int = DEFAULT_BATCH_SIZE,
                 max_tokens: int | None = None):
        options = options if options is not None else Options.defaults(config)
        max_tokens = default_max_tokens() if max_tokens is None else max_tokens
        if batch_size < 1 or max_tokens < 1:
            raise ValueError("batchSize and maxTokens must be >= 1")
        if options.context_length < 1 or options.max_output_patches < 1:
            raise ValueError("contextLength and maxOutputPatches must be >= 1")
        levels = config.quantile_levels()
        for u in options.unrolled_quantiles:
            if not np.any(levels == F32(u)):
                raise ValueError(f"unrolled quantile {float(F32(u))} is not one of the model's levels")
        self.config = config
        self.forward = forward
        self.options = options
        self.batch_size = int(batch_size)
        self.max_tokens = int(max_tokens)

    def with_options(self, o: Options) -> "Chronos2Pipeline":
        return Chronos2Pipeline(self.config, self.forward, o, self.batch_size, self.max_tokens)

    def with_batch_size(self, rows: int) -> "Chronos2Pipeline":
        return Chronos2Pipeline(self.config, self.forward, self.options, rows, self.max_tokens)

    def with_max_tokens(self, tokens: int) -> "Chronos2Pipeline":
        return Chronos2Pipeline(self.config, self.forward, self.options, self.batch_size, tokens)

    # ---- Chronos2Pipeline.forecast (Chronos2Pipeline.java:190-214) ----------------------------

    def forecast(self, series: list, horizon: int) -> list:
        if horizon < 1:
            raise ValueError(f"horizon must be >= 1, got {horizon}")
        ctx = min(self.options.context_length, self.config.context_length)
        prepared = []
        for ts in series:
            if not isinstance(ts, TimeSeries):
                raise ValueError("series must be TimeSeries")
            if ts.has_categorical():
                raise ValueError("Chronos-2 does not support categorical covariates; encode them as numbers")
            prepared.append(self._prepare(ts, horizon, ctx))
        out = []
        start = 0
        while start < len(prepared):  # series join a batch while it has fewer than batch_size rows
            end, rows = start, 0
            while end < len(prepared) and rows < self.batch_size:
                rows += len(prepared[end].context)
                end += 1
            out.extend(self._predict_batch(prepared[start:end], horizon))
            start = end
        return out

    @staticmethod
    def _prepare(ts: TimeSeries, horizon: int, ctx: int) -> _Prepared:
        """Chronos2Pipeline.prepare (Chronos2Pipeline.java:216-243): targets, past covariates, then
        known covariates, each cut to its last min(T, cap) steps; the known covariates' next horizon
        steps as the future, NaN for the other rows."""
        length = ts.length()
        keep = min(length, ctx)
        rows = ts.targets() + ts.past_count() + ts.future_count()
        context = [r[length - keep: length] for r in ts.target]
        context += [r[length - keep: length] for r in (ts.past_covariates or ())]
        future = np.full((rows, horizon), np.nan, F32)
        for v, fc in enumerate(ts.future_covariates or ()):
            if fc.size < length + horizon:
                raise ValueError(f"future covariates need at least {length + horizon} steps, got {fc.size}")
            context.append(fc[length - keep: length])
            future[ts.targets() + ts.past_count() + v] = fc[length: length + horizon]
        return _Prepared(context, future, ts.targets())

    # ---- predictBatch (Chronos2Pipeline.java:245-325) -----------------------------------------

    def _predict_batch(self, batch: list, horizon: int) -> list:
        c = self.config
        length = max(p.context[0].size for p in batch)
        counts = np.array([len(p.context) for p in batch], np.int64)
        n_rows = int(counts.sum())
        first_row = (np.cumsum(counts) - counts).tolist()
        all_rows = [row for p in batch for row in p.context]
        if all(row.size == length for row in all_rows):  # no left padding: one copy
            context = np.stack(all_rows).astype(F32, copy=False)
        else:
            context = np.full((n_rows, length), np.nan, F32)
            for r, row in enumerate(all_rows):
                context[r, length - row.size:] = row
        future = np.concatenate([p.future for p in batch]).astype(F32, copy=False)
        ids = np.zeros(len(batch), np.int32) if self.options.cross_learning else np.arange(len(batch), dtype=np.int32)
        group = np.repeat(ids, counts)
        rows, q = n_rows, c.num_quantiles
        prediction = self._predict_step(context, group, future, self._output_patches(horizon))
        predictions = [prediction]
        remaining = horizon - prediction.shape[2]
        if remaining > 0:
            unrolled = np.asarray(self.options.unrolled_quantiles, F32)
            paths = unrolled.size
            # (row, path) rows; a group mixes only the rows of one path
            context = np.repeat(context, paths, axis=0)
            future = np.repeat(future, paths, axis=0)
            group = (np.repeat(group.astype(np.int64), paths) * paths + np.tile(np.arange(paths), rows)).astype(np.int32)
            path_mass = qm.probability_mass(unrolled)
            level_mass = qm.probability_mass(c.quantile_levels())
            weights = (path_mass[:, None] * level_mass[None, :]).astype(F32).reshape(-1)
            while remaining > 0:
                prediction, context, future = self._unroll(context, group, future, prediction, unrolled, weights,
                                                           self._output_patches(remaining))
                predictions.append(prediction)
                remaining -= prediction.shape[2]
        levels = c.quantile_levels()
        merged = np.concatenate(predictions, axis=2)[:, :, :horizon]
        out = []
        for s, p in enumerate(batch):
            out.append(Forecast(levels, np.ascontiguousarray(merged[first_row[s]: first_row[s] + p.targets], F32)))
        return out

    def _output_patches(self, remaining: int) -> int:
        ps = self.config.patch_size
        return min((remaining + ps - 1) // ps, self.options.max_output_patches)

    def _unroll(self, context, group, future, prediction, unrolled, weights, output_patches: int):
        """_autoregressive_unroll_for_long_horizon (Chronos2Pipeline.java:338-410): each path's
        context extended by its level of the merged forecast, the known covariates slid in, the next
        pass, and its paths * Q forecasts per row merged back into the model's levels."""
        c = self.config
        rows, q, h = prediction.shape
        paths = unrolled.size
        levels = c.quantile_levels()
        values = np.ascontiguousarray(prediction.transpose(0, 2, 1)).reshape(rows * h, q)
        up = qm.interpolate(unrolled, levels, values).reshape(rows, h, paths)
        length = min(context.shape[1] + h, c.context_length)
        ext = np.concatenate([context, up.transpose(0, 2, 1).reshape(rows * paths, h)], axis=1)
        nxt = np.ascontiguousarray(ext[:, ext.shape[1] - length:])
        # _slide_context_and_future_covariates: known future values replace the forecast
        slide = min(h, future.shape[1])
        if slide > 0:
            f = future[:, :slide]
            tail = nxt[:, length - h: length - h + slide]
            nxt[:, length - h: length - h + slide] = np.where(np.isnan(f), tail, f)
        next_future = np.ascontiguousarray(future[:, min(h, future.shape[1]):])
        pred = self._predict_step(nxt, group, next_future, output_patches)
        steps = pred.shape[2]
        samples = pred.reshape(rows, paths, q, steps).transpose(0, 3, 1, 2).reshape(rows * steps, paths * q)
        merged = qm.weighted_quantile(levels, weights, samples)
        out = np.ascontiguousarray(merged.reshape(rows, steps, q).transpose(0, 2, 1), F32)
        return out, nxt, next_future

    def _predict_step(self, context, group, future, output_patches: int) -> np.ndarray:
        """_predict_step (Chronos2Pipeline.java:412-421): the future covariates padded with NaN or cut
        to the forecast, then the model."""
        size = output_patches * self.config.patch_size
        f = np.full((future.shape[0], size), np.nan, F32)
        k = min(size, future.shape[1])
        f[:, :k] = future[:, :k]
        return self._run(ModelInput(np.ascontiguousarray(context, F32), np.ascontiguousarray(group, np.int32), f,
                                    output_patches))

    def _run(self, inp: ModelInput) -> np.ndarray:
        """Chronos2Pipeline.run (Chronos2Pipeline.java:423-448): the pass as several when it holds more
        than max_tokens tokens, whole groups per pass (in order of first appearance), each pass's rows
        in input order; the forecasts are unchanged by the split."""
        c = self.config
        ps = c.patch_size
        per_row = (min(inp.length(), c.context_length) + ps - 1) // ps + (1 if c.use_reg_token else 0) + inp.output_patches
        if per_row * inp.rows() <= self.max_tokens:
            return self._call(inp)
        by_group: dict = {}
        for i, g in enumerate(inp.group.tolist()):
            by_group.setdefault(g, []).append(i)
        out = [None] * inp.rows()
        chunk: list = []
        for members in by_group.values():
            if chunk and (len(chunk) + len(members)) * per_row > self.max_tokens:
                self._run_chunk(inp, chunk, out)
                chunk = []
            chunk.extend(members)
        self._run_chunk(inp, chunk, out)
        return np.stack(out)

    def _run_chunk(self, inp: ModelInput, rows: list, out: list) -> None:
        idx = np.sort(np.asarray(rows, np.int64))
        r = self._call(ModelInput(inp.context[idx], inp.group[idx], inp.future_covariates[idx], inp.output_patches))
        for i, k in enumerate(idx):
            out[k] = r[i]

    def _call(self, inp: ModelInput) -> np.ndarray:
        r = np.asarray(self.forward(inp), F32)
        q, steps = self.config.num_quantiles, inp.output_patches * self.config.patch_size
        if r.shape != (inp.rows(), q, steps):
            raise RuntimeError(f"the forward pass returned {r.shape}, expected {(inp.rows(), q, steps)}")
        return r
