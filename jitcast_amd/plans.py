"""Plans: one captured hipGraph per batch shape, and the cache that keeps them.

The reference compiles one TornadoVM execution plan per input shape and keeps them in a PlanCache
(J/tornado/PlanCache.java:40-161): at most `max_plans`, within `max_bytes` of device memory, least
recently used evicted first, a failed first run retried once after clearing the cache. Here a plan
is a hipGraph captured from the library's entry points (jc_plan_begin / jc_plan_end), replayed with
jc_plan_launch_on; the device buffers a plan adopts are its footprint.
"""
from __future__ import annotations

import ctypes
import threading
from collections import OrderedDict
from contextlib import contextmanager
from typing import Callable, Generic, Hashable, TypeVar

from . import _lib
from .runtime import context


class Plan:
    """A captured, instantiated hipGraph (jc_plan) of one device."""

    def __init__(self, handle: ctypes.c_void_p, device: int = 0, ctx=None):
        self.handle = handle
        self.device = device
        self._ctx = ctx  # the capturing context: the plan refers to it, so it must outlive the plan

    def launch(self) -> None:
        """Replays the graph on torch's current stream (jc_plan_launch_on), from any thread: the
        plan keeps the context of the thread that captured it, and that context's binding is
        neither read nor changed."""
        import torch

        stream = torch.cuda.current_stream(self.device).cuda_stream
        _lib.call("jc_plan_launch_on", self.handle, ctypes.c_void_p(stream))

    def adopt(self, dptr: int, nbytes: int) -> None:
        """Hands a jc_alloc buffer to the plan: freed by close(), counted by device_bytes()."""
        _lib.call("jc_plan_adopt", self.handle, ctypes.c_void_p(dptr), nbytes)

    def device_bytes(self) -> int:
        return int(_lib.lib().jc_plan_device_bytes(self.handle)) if self.handle else 0

    @property
    def key(self) -> int:
        return int(_lib.lib().jc_plan_key(self.handle))

    def close(self) -> None:
        if self.handle:
            h, self.handle = self.handle, None
            _lib.call("jc_plan_destroy", h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@contextmanager
def capture(shape_key: int, device: int = 0):
    """Captures the entry points called inside the block (on torch's current stream, which must
    not be the null stream) into a Plan, yielded as a one-element list filled on exit."""
    ctx = context(device)
    _lib.call("jc_plan_begin", ctx.handle, ctypes.c_uint64(shape_key))
    box: list[Plan] = []
    try:
        yield box
    finally:
        h = ctypes.c_void_p()
        _lib.call("jc_plan_end", ctx.handle, ctypes.byref(h))
        box.append(Plan(h, device, ctx))


K = TypeVar("K", bound=Hashable)
P = TypeVar("P")


class PlanCache(Generic[K, P]):
    """PlanCache.run's contract (PlanCache.java:70-100): plans keyed by shape, LRU within a count
    and byte budget, one lock around every call; a plan whose first use fails is closed, and if
    other plans were cached they are all closed and the plan is built and used once more."""

    def __init__(self, max_plans: int, max_bytes: int):
        if max_plans < 1 or max_bytes < 1:
            raise ValueError("a plan cache needs room for one plan")
        self.max_plans = max_plans
        self.max_bytes = max_bytes
        self._plans: OrderedDict = OrderedDict()  # key -> (plan, bytes), least recent first
        self._bytes = 0
        self._lock = threading.RLock()

    def run(self, key: K, build: Callable[[K], P], use: Callable[[P], object]):
        with self._lock:
            if key in self._plans:
                self._plans.move_to_end(key)
                return use(self._plans[key][0])
            self._evict_while(lambda: len(self._plans) >= self.max_plans)
            plan = build(key)
            try:
                result = use(plan)
            except Exception as first:
                _close_quietly(plan, first)
                if not self._plans:
                    raise
                self._clear(first)
                plan = build(key)
                try:
                    result = use(plan)
                except Exception as second:
                    second.__context__ = first
                    _close_quietly(plan, second)
                    raise
            nbytes = plan.device_bytes()
            self._evict_while(lambda: bool(self._plans) and self._bytes + nbytes > self.max_bytes)
            self._plans[key] = (plan, nbytes)
            self._bytes += nbytes
            return result

    def keys(self) -> list:
        """The shapes cached, least recently used first."""
        with self._lock:
            return list(self._plans)

    def cached_bytes(self) -> int:
        with self._lock:
            return self._bytes

    def _evict_while(self, full) -> None:
        while full() and self._plans:
            _, (plan, nbytes) = self._plans.popitem(last=False)
            self._bytes -= nbytes
            plan.close()

    def _clear(self, failure: BaseException) -> None:
        plans = [p for p, _ in self._plans.values()]
        self._plans.clear()
        self._bytes = 0
        for p in plans:
            _close_quietly(p, failure)

    def close(self) -> None:
        """Closes every plan, even when some fail; the first failure is raised."""
        with self._lock:
            plans = [p for p, _ in self._plans.values()]
            self._plans.clear()
            self._bytes = 0
            first = None
            for p in plans:
                try:
                    p.close()
                except Exception as e:  # noqa: PERF203
                    if first is None:
                        first = e
            if first is not None:
                raise first


def _close_quietly(plan, failure: BaseException) -> None:
    try:
        plan.close()
    except Exception as e:
        failure.__context__ = failure.__context__ or e
