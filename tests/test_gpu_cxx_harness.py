"""The C++ caller of the ABI (tests/cxx/abi_harness.cpp): a program linked against libjitcast_hip.so
and the CPU oracle, with no Python between it and the library. On the GPU it checks time attention
(with the folded last query), group attention, jc_linear, a captured plan and the error codes against
the oracle; on the CPU, that it is built and resolves the in-tree libraries."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HARNESS = ROOT / "tests" / "cxx" / "abi_harness"


def test_harness_is_built_against_the_in_tree_libraries():
    assert HARNESS.exists(), "build with __graft_entry__.build() (make -C tests/cxx)"
    out = subprocess.run(["ldd", str(HARNESS)], capture_output=True, text=True, check=True).stdout
    found = {l.split()[0]: Path(l.split("=>")[1].split("(")[0].strip()).resolve()
             for l in out.splitlines() if "=>" in l}
    assert found["libjitcast_hip.so"] == ROOT / "jitcast_amd" / "libjitcast_hip.so"
    assert found["libjc_oracle.so"] == ROOT / "oracle" / "libjc_oracle.so"


@pytest.mark.gpu
def test_harness_passes_on_the_gpu():
    print("case C++ ABI harness", flush=True)
    r = subprocess.run([str(HARNESS)], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi harness: all checks passed" in r.stdout
