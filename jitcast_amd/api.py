"""The model-independent forecasting API: series in, quantiles out (J/api).

  TimeSeries      one input: target rows plus optional covariates, NaN where missing, shapes
                  checked when built (J/api/TimeSeries.java:30-151)
  Forecast        the quantile levels and values[target][level][step] of one series
                  (J/api/Forecast.java:26-52)
  ForecastEngine  forecast(series, horizon) / name() / close(), closable more than once, usable as
                  a context manager (J/api/ForecastEngine.java:37-57)

Errors are the reference's IllegalArgumentExceptions as ValueError.
"""
from __future__ import annotations

import abc
import math
from dataclasses import dataclass

import numpy as np


def _rows(a, what: str):
    """A [rows][steps] float input as a list of float32 rows (rows may differ in length)."""
    if a is None:
        return None
    if isinstance(a, np.ndarray) and a.ndim == 2:
        return [np.ascontiguousarray(r, np.float32) for r in a]
    out = [np.ascontiguousarray(np.asarray(r, np.float32).reshape(-1)) for r in a]
    return out


@dataclass(frozen=True, init=False)
class TimeSeries:
    """target [V_t][T]; past_covariates [V_p][T] or None; future_covariates [V_f][>= T + H] or
    None (extra trailing steps are ignored); past_categorical [C_p][T] and future_categorical
    [C_f][>= T + H] category codes (finite or NaN), or None."""

    target: tuple
    past_covariates: tuple | None
    future_covariates: tuple | None
    past_categorical: tuple | None
    future_categorical: tuple | None

    def __init__(self, target, past_covariates=None, future_covariates=None, past_categorical=None,
                 future_categorical=None):
        tgt = _rows(target, "target")
        if not tgt:
            raise ValueError("a series needs at least one target row")
        t = tgt[0].size
        if t == 0:
            raise ValueError("a series needs at least one time step")
        for r in tgt:
            _require_length(r.size, t, "target")
        past = _rows(past_covariates, "past covariate")
        for r in past or ():
            _require_length(r.size, t, "past covariate")
        fut = _rows(future_covariates, "future covariate")
        for r in fut or ():
            if r.size < t:
                raise ValueError("a future covariate row is shorter than the target")
        pcat = None if past_categorical is None else [np.asarray(r, np.float64).reshape(-1) for r in past_categorical]
        for r in pcat or ():
            _require_length(r.size, t, "past categorical covariate")
            _require_not_infinite(r)
        fcat = None if future_categorical is None else [np.asarray(r, np.float64).reshape(-1) for r in future_categorical]
        for r in fcat or ():
            if r.size < t:
                raise ValueError("a future categorical covariate row is shorter than the target")
            _require_not_infinite(r)
        tup = lambda x: None if x is None else tuple(x)  # noqa: E731
        object.__setattr__(self, "target", tuple(tgt))
        object.__setattr__(self, "past_covariates", tup(past))
        object.__setattr__(self, "future_covariates", tup(fut))
        object.__setattr__(self, "past_categorical", tup(pcat))
        object.__setattr__(self, "future_categorical", tup(fcat))

    @staticmethod
    def univariate(values) -> "TimeSeries":
        """A series with one target row and no covariates."""
        return TimeSeries([values])

    def length(self) -> int:
        return int(self.target[0].size)

    def targets(self) -> int:
        return len(self.target)

    def past_count(self) -> int:
        return 0 if self.past_covariates is None else len(self.past_covariates)

    def future_count(self) -> int:
        return 0 if self.future_covariates is None else len(self.future_covariates)

    def past_categorical_count(self) -> int:
        return 0 if self.past_categorical is None else len(self.past_categorical)

    def future_categorical_count(self) -> int:
        return 0 if self.future_categorical is None else len(self.future_categorical)

    def has_categorical(self) -> bool:
        return self.past_categorical_count() + self.future_categorical_count() > 0

    def rows(self) -> int:
        """The rows the series contributes to a forward pass: targets and all covariates."""
        return (self.targets() + self.past_count() + self.future_count() + self.past_categorical_count()
                + self.future_categorical_count())


def _require_length(length: int, t: int, what: str) -> None:
    if length != t:
        raise ValueError(f"every {what} row must have the target's length {t}")


def _require_not_infinite(codes: np.ndarray) -> None:
    if np.isinf(codes).any():
        raise ValueError("category codes must be finite or NaN")


@dataclass(frozen=True)
class Forecast:
    """levels: ascending quantile levels (float32); values: float32 [targets][levels][horizon]."""

    levels: np.ndarray
    values: np.ndarray

    def targets(self) -> int:
        return int(self.values.shape[0])

    def horizon(self) -> int:
        return int(self.values.shape[2])

    def median(self, t: int) -> np.ndarray:
        """The 0.5 level of target t."""
        for q, lv in enumerate(self.levels):
            if math.fabs(float(lv) - 0.5) < 1e-6:
                return self.values[t][q]
        raise RuntimeError("no 0.5 quantile level")


class ForecastEngine(abc.ABC):
    """A forecasting engine for one model family. Calls from several threads run one at a time;
    close() releases device memory and may be called more than once."""

    @abc.abstractmethod
    def forecast(self, series: list, horizon: int) -> list:
        """One Forecast per series, in order. ValueError if horizon < 1 or a series has inputs the
        model does not take."""

    @abc.abstractmethod
    def name(self) -> str:
        """A short name for logs and benchmark records."""

    @abc.abstractmethod
    def close(self) -> None:
        """Releases the engine's device memory and weights; later calls do nothing."""

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False
