"""Engines used from several threads (ForecastEngine.java:33-35: an engine can be shared between
threads, and the reference's PlanCache.run serialises its calls, PlanCache.java:70). Each thread
keeps its own device context (its own stream binding and hipBLASLt handle), and a plan replays on the
caller's stream (jc_plan_launch_on), so a Chronos-2 engine with plans and a Timestral engine
forecasting at the same time on two threads, and one engine shared by two threads, give exactly the
forecasts of a single-threaded run."""
import threading

import numpy as np
import pytest

from jitcast_amd import checkpoint as ck
from jitcast_amd import timestral_model as tm
from jitcast_amd.api import TimeSeries
from jitcast_amd.chronos2_model import random_weights
from jitcast_amd.engine import HipChronos2Engine, HipTimestralEngine
from tests.test_gpu_engine import C as C2
from tests.test_gpu_ts_engine import C as CTS
from tests.test_pipeline import _mixed_batch
from tests.test_ts_pipeline import _series

pytestmark = pytest.mark.gpu


def _run_threads(jobs, timeout=240.0):
    """jobs: (name, callable); each runs on its own thread. Returns {name: [results]}."""
    results, errors = {}, []

    def body(name, fn):
        try:
            results[name] = fn()
        except BaseException as e:  # noqa: BLE001 (reported below)
            errors.append((name, e))

    threads = [threading.Thread(target=body, args=(n, f), daemon=True) for n, f in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout)
        assert not t.is_alive(), "a forecasting thread did not finish"
    assert not errors, errors
    return results


def _same(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x.values, y.values)


def test_two_engines_on_two_threads(gpu, tmp_path):
    print("case two engines (chronos-2 bf16 with plans, timestral f32) on two threads", flush=True)
    c2_dir, ts_dir = tmp_path / "c2", tmp_path / "ts"
    ck.write_chronos2(c2_dir, C2, random_weights(C2, seed=21, std=0.1))
    ck.write_timestral(ts_dir, CTS, tm.random_weights(CTS, seed=31, std=0.1))
    c2_series = [TimeSeries(t, p, k) for t, p, k in _mixed_batch(11, 25, 100)]
    ts_series = _series()
    with HipChronos2Engine.load(c2_dir, dtype="bf16", max_plans=4) as e1, \
            HipTimestralEngine.load(ts_dir, dtype="f32") as e2:
        ref1 = e1.forecast(c2_series, 100)
        ref2 = e2.forecast(ts_series, 40)
        out = _run_threads([("c2", lambda: [e1.forecast(c2_series, 100) for _ in range(4)]),
                            ("ts", lambda: [e2.forecast(ts_series, 40) for _ in range(4)])])
        for got in out["c2"]:
            _same(got, ref1)
        for got in out["ts"]:
            _same(got, ref2)
        # one engine shared by two threads: its calls run one at a time, on each caller's stream
        out = _run_threads([(f"t{i}", lambda: [e1.forecast(c2_series, 100) for _ in range(3)]) for i in range(2)])
        for res in out.values():
            for got in res:
                _same(got, ref1)
