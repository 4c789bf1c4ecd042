"""Builds libjitcast_hip.so in-tree with hipcc for gfx950.

Every HIP source under csrc/ is compiled with -Xclang -target-feature -Xclang -packed-fp32-ops
(no packed FP32 VALU code is generated; hipcc's host pass warns that it does not know the
feature, which is harmless) and linked into jitcast_amd/libjitcast_hip.so, which travels with
the source tree to the GPU box.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "_build"
LIB = HERE / "libjitcast_hip.so"
ARCH = os.environ.get("JITCAST_HIP_ARCH", "gfx950")

SOURCES = ["jc_abi.cpp", "jc_blas.cpp", "jc_host.cpp", "ts_host.cpp", "time_attention_f32.hip", "time_attention_lp.hip", "time_attention_lpw.hip", "time_attention_lpp.hip", "time_attention_lps.hip", "gate.hip", "group_attention_f32.hip", "stage_f32.hip", "stage_lp.hip", "c2_tokens.hip", "c2_prep.hip", "ts_block.hip", "ts_ends.hip", "rng.hip"]

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the softmax and rescale read them with VALU ops, which cannot
    # address AGPRs (the AGPR form costs a v_accvgpr copy per element per block)
    "-mllvm", "--amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP extension cannot be built")


def _compile(src: str) -> Path:
    obj = OUT_DIR / (src.replace(".", "_") + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else ["-x", "hip"]
    cmd = [hipcc(), *COMMON, *lang, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    OUT_DIR.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    # hipBLASLt runs the plain GEMMs (jc_blas.cpp); the RPATH finds it where ROCm installs it
    rocm_lib = str(Path(hipcc()).resolve().parent.parent / "lib")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), f"-L{rocm_lib}",
           "-lhipblaslt", f"-Wl,-rpath,{rocm_lib}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
