"""jitcast_amd: an MI355X-native (gfx950) encoder self-attention path for jitCast's
Chronos-2 and Timestral engines, exported as the C ABI libjitcast_hip (include/jitcast_hip.h).

Importing the package loads the library and fails loudly if it is not built: there is no CPU or
PyTorch fallback on the product path.
"""
from . import _lib
from ._lib import JitcastArgumentError, JitcastError, LibraryMissing

_lib.lib()

from . import chronos2, plans, rng, runtime, timestral  # noqa: E402

__all__ = ["chronos2", "timestral", "plans", "rng", "runtime", "JitcastError", "JitcastArgumentError", "LibraryMissing"]
