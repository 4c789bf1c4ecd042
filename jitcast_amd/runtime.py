"""The device context: one jc_ctx per device and thread, launching on torch's current stream.

PyTorch is plumbing here (device memory and streams); every computation on the attention path
runs in libjitcast_hip.
"""
from __future__ import annotations

import ctypes
import sys
import threading
from contextlib import contextmanager

from . import _lib


class HipContext:
    """jc_init/jc_destroy around one device (J/tornado/Devices.java:44-73 picks the device)."""

    def __init__(self, device: int = 0):
        handle = ctypes.c_void_p()
        _lib.call("jc_init", device, ctypes.byref(handle))
        self.handle = handle
        self.device = device

    def bind_torch_stream(self) -> None:
        """Launch on torch's current stream on this device, so launches order with torch work."""
        import torch

        stream = torch.cuda.current_stream(self.device).cuda_stream
        _lib.call("jc_set_stream", self.handle, ctypes.c_void_p(stream))

    def sync(self) -> None:
        _lib.call("jc_sync", self.handle)

    def profile(self, on: bool) -> None:
        """Starts (or restarts) or stops per-kernel timing on this context (jc_profile)."""
        _lib.call("jc_profile", self.handle, 1 if on else 0)

    def profile_report(self) -> str:
        """The kernels timed since profiling started or the last report, one line each (jc_profile_report)."""
        buf = ctypes.create_string_buffer(1 << 16)
        _lib.call("jc_profile_report", self.handle, buf, len(buf))
        return buf.value.decode()

    def device_info(self) -> tuple[int, str]:
        cus = ctypes.c_int()
        arch = ctypes.create_string_buffer(64)
        _lib.call("jc_device_info", self.handle, ctypes.byref(cus), arch, 64)
        return cus.value, arch.value.decode()

    def close(self) -> None:
        if self.handle:
            _lib.lib().jc_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_local = threading.local()


def context(device: int = 0) -> HipContext:
    """The calling thread's context on a device, bound to torch's current stream on every call.

    Each thread keeps its own jc_ctx (its own stream binding and hipBLASLt handle), so engines used
    from different threads never launch on each other's streams: a context's binding only changes
    between the calls of the one thread that owns it."""
    ctxs = getattr(_local, "ctxs", None)
    if ctxs is None:
        ctxs = _local.ctxs = {}
    ctx = ctxs.get(device)
    if ctx is None:
        ctx = ctxs[device] = HipContext(device)
    ctx.bind_torch_stream()
    return ctx


@contextmanager
def kernel_profile(device: int, label: str, on: bool):
    """Per-kernel times of the launches made inside the block, printed to stderr after it: the
    counterpart of the reference's -D<model>.tornado.profile console profiler
    (J/chronos2/tornado/Chronos2Forward.java:301-303). Does nothing when off, or while the current
    stream is being captured into a plan (a capture records no events)."""
    import torch

    if not on or torch.cuda.is_current_stream_capturing():
        yield
        return
    ctx = context(device)
    ctx.profile(True)
    try:
        yield
        report = context(device).profile_report()
        print(f"[{label}]\n{report}", file=sys.stderr, end="", flush=True)
    finally:
        ctx.profile(False)


def timed_replay(label: str, on: bool, replay) -> None:
    """Runs replay(); when on, times it with HIP events on the current stream and prints the time to
    stderr (a captured plan replays as one graph, so its kernels are not timed one by one)."""
    if not on:
        replay()
        return
    import torch

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    replay()
    b.record()
    b.synchronize()
    print(f"[{label}] plan replay {a.elapsed_time(b):.4f} ms", file=sys.stderr, flush=True)


def fill_normal(t, stream_seed: int, mean: float = 0.0, std: float = 1.0) -> None:
    """Fills a float32 CUDA tensor in place with the portable RNG (jc_fill_normal)."""
    ctx = context(t.device.index or 0)
    _lib.call("jc_fill_normal", ctx.handle, ctypes.c_void_p(t.data_ptr()), t.numel(), stream_seed,
              ctypes.c_float(mean), ctypes.c_float(std))


def fill_uniform(t, stream_seed: int, lo: float = 0.0, hi: float = 1.0) -> None:
    ctx = context(t.device.index or 0)
    _lib.call("jc_fill_uniform", ctx.handle, ctypes.c_void_p(t.data_ptr()), t.numel(), stream_seed,
              ctypes.c_float(lo), ctypes.c_float(hi))
