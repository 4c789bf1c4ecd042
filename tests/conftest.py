import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")
    config.addinivalue_line("markers", "slow: a larger case (still minutes at most)")


def pytest_collection_modifyitems(config, items):
    # GPU tests first make sure the library is the HIP build, never a fallback
    pass


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def gpu():
    """The device context; a GPU test fails (not skips) when the library or the GPU is missing."""
    import torch

    import jitcast_amd

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    ctx = jitcast_amd.runtime.context(0)
    cus, arch = ctx.device_info()
    print(f"[gpu] {arch} with {cus} CUs", flush=True)
    return ctx


@pytest.fixture(params=["stream", "wide", "persist"])
def lp_kernel(request, monkeypatch):
    """Which bf16/fp16 time-attention kernel the library launches (JITCAST_HIP_LP_KERNEL): the
    streaming one, the row-wide one (rows of 256+ tokens and head width 32 or 64) or the persistent
    ones (Chronos-2, head width 64: rows of 257..513 tokens, and the short-row kernel for rows of
    65..160); a shape the chosen kernel does not take falls back to the row-wide or streaming kernel. Unset, Chronos-2 uses the persistent kernel
    where it fits, Timestral the streaming one."""
    monkeypatch.setenv("JITCAST_HIP_LP_KERNEL", request.param)
    return request.param


@pytest.fixture(scope="session", autouse=True)
def _built_library():
    """CPU tests load libjitcast_hip (symbols, host helpers); build it once if this tree has none."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("jitcast_amd_build", ROOT / "jitcast_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    if not b.LIB.exists():
        b.build(verbose=False)


@pytest.fixture(params=["blas", "own"])
def gemm_path(request, monkeypatch):
    """Which kernels run the plain GEMMs (JITCAST_HIP_GEMM): hipBLASLt (the default) or the library's
    own MFMA kernels (gemm_f32, gemm_lp), which also take the combinations hipBLASLt declines."""
    if request.param == "own":
        monkeypatch.setenv("JITCAST_HIP_GEMM", "own")
    else:
        monkeypatch.delenv("JITCAST_HIP_GEMM", raising=False)
    return request.param
