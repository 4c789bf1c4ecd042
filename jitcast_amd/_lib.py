"""ctypes binding of libjitcast_hip (include/jitcast_hip.h).

The library is the product: there is no fallback. If it is not built, loading raises
LibraryMissing naming the build command.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libjitcast_hip.so"
HEADER = HERE.parent / "include" / "jitcast_hip.h"

JC_OK, JC_EINVAL, JC_EHIP, JC_ENOMEM, JC_EUNSUPPORTED, JC_ESTATE = 0, -1, -2, -3, -4, -5
JC_F32, JC_BF16, JC_F16, JC_F16X3 = 0, 1, 2, 3


class LibraryMissing(ImportError):
    pass


class JitcastError(RuntimeError):
    """A non-zero jc_status; `code` is the status, the message is jc_last_error()."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class JitcastArgumentError(JitcastError, ValueError):
    """JC_EINVAL: the reference throws IllegalArgumentException for these."""


_c = ctypes
_vp, _i, _f, _sz, _i64 = _c.c_void_p, _c.c_int, _c.c_float, _c.c_size_t, _c.c_int64
_i32p = _c.c_void_p  # device int32 pointers are passed as addresses

# name -> (restype, argtypes); every function the header declares must be listed here
SIGNATURES = {
    "jc_init": (_i, [_i, _c.POINTER(_vp)]),
    "jc_destroy": (_i, [_vp]),
    "jc_set_stream": (_i, [_vp, _vp]),
    "jc_stream": (_vp, [_vp]),
    "jc_alloc": (_i, [_vp, _sz, _c.POINTER(_vp)]),
    "jc_free": (_i, [_vp, _vp]),
    "jc_memcpy_h2d": (_i, [_vp, _vp, _vp, _sz]),
    "jc_memcpy_d2h": (_i, [_vp, _vp, _vp, _sz]),
    "jc_memcpy_d2d": (_i, [_vp, _vp, _vp, _sz]),
    "jc_sync": (_i, [_vp]),
    "jc_device_info": (_i, [_vp, _c.POINTER(_i), _c.c_char_p, _sz]),
    "jc_last_error": (_c.c_char_p, []),
    "jc_version": (_i, []),
    "jc_plan_begin": (_i, [_vp, _c.c_uint64]),
    "jc_plan_end": (_i, [_vp, _c.POINTER(_vp)]),
    "jc_plan_launch": (_i, [_vp]),
    "jc_plan_launch_on": (_i, [_vp, _vp]),
    "jc_profile": (_i, [_vp, _i]),
    "jc_profile_report": (_i, [_vp, _c.c_char_p, _sz]),
    "jc_plan_adopt": (_i, [_vp, _vp, _sz]),
    "jc_plan_device_bytes": (_c.c_int64, [_vp]),
    "jc_plan_key": (_c.c_uint64, [_vp]),
    "jc_plan_destroy": (_i, [_vp]),
    "jc_fill_normal": (_i, [_vp, _vp, _c.c_uint64, _c.c_uint64, _f, _f]),
    "jc_fill_uniform": (_i, [_vp, _vp, _c.c_uint64, _c.c_uint64, _f, _f]),
    "jc_c2_rope_table": (_i, [_i, _i, _f, _vp]),
    "jc_c2_time_attention": (_i, [_vp, _vp, _vp, _i32p, _vp, _i, _i, _i, _i, _i, _i]),
    "jc_c2_group_attention": (_i, [_vp, _vp, _vp, _i32p, _i32p, _i32p, _i, _i, _i, _i, _i, _i]),
    "jc_ts_rope_table": (_i, [_i, _i, _i, _i, _f, _vp]),
    "jc_ts_time_attention": (_i, [_vp, _vp, _vp, _i32p, _i32p, _i32p, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i]),
    "jc_ts_gate": (_i, [_vp, _vp, _vp, _c.c_int64, _i]),
    "jc_ts_variate_attention": (_i, [_vp, _vp, _vp, _i32p, _i32p, _i32p, _i32p, _i, _vp, _i, _i, _i, _i, _i, _i, _i]),
    "jc_c2_live": (_i, [_vp, _i, _i, _i, _i, _i, _vp]),
    "jc_c2_group_order": (_i, [_vp, _i, _vp, _c.POINTER(_i)]),
    "jc_c2_group_bounds": (_i, [_vp, _i, _vp, _vp]),
    "jc_linear": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "jc_rms_norm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f]),
    "jc_c2_layer_workspace_bytes": (_c.c_int64, [_i, _i, _i, _i, _i, _i]),
    "jc_c2_layer": (_i, [_vp, _vp, _vp, _i32p, _vp, _i32p, _i32p, _vp, _i, _i, _i, _i, _i, _i, _f, _i]),
    "jc_c2_layer_static": (_i, [_vp, _vp, _vp, _i32p, _vp, _i32p, _i32p, _i, _i, _i, _i, _i, _i, _f, _i]),
    "jc_linear_lp": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i]),
    "jc_rms_norm_lp": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _i]),
    "jc_to_lp": (_i, [_vp, _vp, _vp, _c.c_int64, _i]),
    "jc_split_f16x3": (_i, [_vp, _vp, _i, _vp, _i, _i, _i]),
    "jc_c2_assemble": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "jc_c2_gather_future": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "jc_ts_residual": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "jc_ts_assemble": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "jc_ts_gather_decoder": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "jc_swiglu": (_i, [_vp, _vp, _vp, _i64, _i, _i]),
    "jc_ts_prep": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _f, _i, _vp, _vp, _vp, _vp]),
    "jc_ts_finish": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _i, _i, _vp]),
    "jc_c2_prep": (_i, [_vp, _vp, _i64, _i, _vp, _i64, _i, _vp, _i, _i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _vp]),
    "jc_c2_finish": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "jc_c2_residual": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "jc_ts_block_layout": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _c.POINTER(_i), _c.POINTER(_i), _vp,
                                _vp, _vp]),
    "jc_ts_context_stats": (_i, [_vp, _vp, _i, _i, _f, _vp, _vp, _vp, _vp]),
    "jc_ts_advancing_frames": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _f, _vp, _vp]),
}

_lib = None


def header_symbols() -> list[str]:
    """The function names include/jitcast_hip.h declares."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jc_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = Path(os.environ.get("JITCAST_HIP_LIB", LIB_PATH))
        if not path.exists():
            raise LibraryMissing(
                f"{path} is not built; run `python jitcast_amd/build.py` (or __graft_entry__.build())")
        # One HIP runtime per process: torch ships libamdhip64.so with SONAME libamdhip64.so.7. Loading
        # torch first lets the dynamic loader resolve this library's libamdhip64.so.7 to that same
        # copy, so device pointers and streams are shared. Without torch, /opt/rocm's runtime loads.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().jc_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc == JC_OK:
        return
    msg = last_error()
    if rc == JC_EINVAL:
        raise JitcastArgumentError(rc, msg)
    raise JitcastError(rc, msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
