"""Strict option readers, as the reference's -D properties (J/util/Options.java:38-146).

The properties come from the environment variable JITCAST_OPTS, written as Java flags
("-Dchronos2.maxTokens=65536 -Dchronos2.hip.dtype=bf16"), and from set_property (System.setProperty).
A blank value is unset. A value that does not parse fails with the property's name and what was
expected; unknown properties are ignored, as the JVM ignores them.

Properties read by this package:
  chronos2.maxTokens        tokens per forward pass before the pipeline splits it (131072)
  chronos2.hip.dtype        f32 | bf16 | fp16 | f16x3: the encoder's GEMM and time-attention type;
                            f16x3 keeps fp32 results with the GEMMs on three-term fp16 splits (f32)
  chronos2.hip.plans        plans cached per engine, one hipGraph per batch shape; 0 runs eagerly (8)
  chronos2.hip.planBytes    device bytes the cached plans may hold (the device's memory)
  chronos2.hip.profile      print per-kernel times of each eager forward and the time of each plan
                            replay to stderr, as -Dchronos2.tornado.profile (false)
  timestral.maxTokens       tokens (rows x patches) per Timestral forward pass before the pipeline
                            splits a call into windows (131072)
  timestral.hip.dtype       f32 | bf16 | fp16 | f16x3: the Timestral engine's GEMM and attention type (f32;
                            f16x3: fp32 activations, each GEMM over three-term fp16 splits)
  timestral.hip.buckets     pad blocks to shared shapes before the forward (true)
  timestral.hip.plans       plans cached per HipTimestralModel, one hipGraph per block shape; 0 runs
                            eagerly (8)
  timestral.hip.planBytes   device bytes those plans may hold (the device's memory)
  timestral.hip.profile     as chronos2.hip.profile, for the Timestral block (false)
  jitcast.hip.device        the GPU an engine runs on (0)
"""
from __future__ import annotations

import os
import shlex
import threading

_lock = threading.Lock()
_set: dict = {}


def _env_properties() -> dict:
    props = {}
    for tok in shlex.split(os.environ.get("JITCAST_OPTS", "")):
        if tok.startswith("-D") and "=" in tok:
            k, v = tok[2:].split("=", 1)
            props[k] = v
        elif tok.startswith("-D"):
            props[tok[2:]] = ""
    return props


def set_property(name: str, value: str | None) -> None:
    """Sets (or with None clears) a property for this process, over JITCAST_OPTS."""
    with _lock:
        if value is None:
            _set.pop(name, None)
        else:
            _set[name] = str(value)


def _raw(name: str):
    with _lock:
        v = _set.get(name)
    if v is None:
        v = _env_properties().get(name)
    if v is None or not v.strip():
        return None
    return v.strip()


def _bad(name: str, value: str, expected: str) -> ValueError:
    return ValueError(f"-D{name}={value}: expected {expected}")


def _parse_int(v: str, lo: int, hi: int):
    # Java's parseInt/parseLong: an optional sign and decimal digits only
    s = v[1:] if v[:1] in "+-" else v
    if not s or not s.isdigit() or not s.isascii():
        return None
    i = int(v)
    return i if lo <= i <= hi else None


def integer(name: str, default: int, minimum: int) -> int:
    """Options.integer: a 32-bit integer of at least minimum."""
    v = _raw(name)
    if v is None:
        return default
    i = _parse_int(v, -(1 << 31), (1 << 31) - 1)
    if i is not None and i >= minimum:
        return i
    raise _bad(name, v, f"an integer of at least {minimum}")


def number(name: str, default: int, minimum: int) -> int:
    """Options.number: a 64-bit whole number of at least minimum."""
    v = _raw(name)
    if v is None:
        return default
    i = _parse_int(v, -(1 << 63), (1 << 63) - 1)
    if i is not None and i >= minimum:
        return i
    raise _bad(name, v, f"a whole number of at least {minimum}")


_UNITS = (("TB", 1 << 40), ("GB", 1 << 30), ("MB", 1 << 20), ("KB", 1 << 10), ("B", 1))


def parse_bytes(text: str) -> int:
    """Options.parseBytes: a whole number with an optional B/KB/MB/GB/TB suffix; -1 if it does not
    parse or overflows 64 bits."""
    s = text.strip().upper()
    unit = 1
    for suffix, mult in _UNITS:
        if s.endswith(suffix):
            unit = mult
            s = s[: -len(suffix)].strip()
            break
    i = _parse_int(s, -(1 << 63), (1 << 63) - 1)
    if i is None:
        return -1
    b = i * unit
    return b if -(1 << 63) <= b < (1 << 63) else -1


def bytes_(name: str, default: int, minimum: int) -> int:
    """Options.bytes: a size such as 512MB or 8GB, at least minimum bytes."""
    v = _raw(name)
    if v is None:
        return default
    b = parse_bytes(v)
    if b < minimum:
        raise _bad(name, v, f"a size of at least {minimum} bytes, such as 512MB or 8GB")
    return b


def boolean(name: str, default: bool) -> bool:
    """Options.bool: true or false, any case."""
    v = _raw(name)
    if v is None:
        return default
    if v.lower() == "true":
        return True
    if v.lower() == "false":
        return False
    raise _bad(name, v, "true or false")


def choice(name: str, default: str, *allowed: str) -> str:
    """Options.choice: one of allowed, any case; returns the allowed spelling."""
    v = _raw(name)
    if v is None:
        return default
    for a in allowed:
        if a.lower() == v.lower():
            return a
    raise _bad(name, v, "one of " + ", ".join(allowed))
