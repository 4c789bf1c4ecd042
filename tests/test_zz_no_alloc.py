"""jc_c2_layer_static (the allocation-free layer) against jc_c2_layer with a caller workspace, through
the C ABI, two calls in a row on the static scratch (the second with a smaller input), in fp32, bf16
and f16x3 (three-term fp16 splits, fp32 results). The static layer runs its GEMMs on the library's
own kernels (no library routine that could allocate): against jc_c2_layer on those same kernels
(JITCAST_HIP_GEMM=own) it agrees bit for bit, against jc_c2_layer on its default GEMMs (hipBLASLt)
within the parity bars (1e-4 fp32 and f16x3; bf16 to the rounding of its storage type). A call past
the scratch's size is rejected before any launch."""
import numpy as np
import pytest
import torch

from jitcast_amd import chronos2
from jitcast_amd._lib import JitcastArgumentError

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
D, HEADS, DH, DFF = 256, 4, 64, 512


def _weights(dtype_code: int, seed: int = 0) -> dict:
    g = torch.Generator().manual_seed(seed)
    inner = HEADS * DH
    shapes = {"time_qkv": (3 * inner, D), "time_o": (D, inner), "group_qkv": (3 * inner, D), "group_o": (D, inner),
              "wi": (DFF, D), "wo": (D, DFF)}
    w = {}
    for k, s in shapes.items():
        t = (0.05 * torch.randn(s, generator=g)).to(DEV)
        if dtype_code == chronos2._lib.JC_F16X3:
            x3 = torch.empty(s[0], 3 * s[1], dtype=torch.float16, device=DEV)
            chronos2.split_f16x3(t, x3, weights=True)
            t = x3
        elif dtype_code != chronos2._lib.JC_F32:
            lp = torch.empty(s, dtype=torch.bfloat16, device=DEV)
            chronos2.to_lp(t, lp)
            t = lp
        w[k] = t
    for k in ("time_norm", "group_norm", "mlp_norm"):
        w[k] = (1 + 0.05 * torch.randn(D, generator=g)).to(DEV)
    w["wi_bias"] = (0.05 * torch.randn(DFF, generator=g)).to(DEV)
    return w


def _inputs(rows: int, n: int, per_group: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows * n, D, generator=g).to(DEV)
    live = torch.ones(rows, n, dtype=torch.int32)
    for r in range(rows):
        live[r, : (7 * r) % (n // 2)] = 0
    group = np.arange(rows, dtype=np.int32) // per_group
    gs, ge = chronos2.group_bounds(group)
    table = torch.from_numpy(chronos2.rope_table(n, DH)).to(DEV)
    return x, live.reshape(-1).to(DEV), table, torch.from_numpy(gs).to(DEV), torch.from_numpy(ge).to(DEV)


def _rel(a, b):
    return float((a.double() - b.double()).abs().max() / b.double().abs().max())


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16x3"])
def test_static_layer_matches_workspace_layer(gpu, dt, monkeypatch):
    code = {"f32": chronos2._lib.JC_F32, "bf16": chronos2._lib.JC_BF16, "f16x3": chronos2._lib.JC_F16X3}[dt]
    w = _weights(code)
    for call, (rows, n, per_group) in enumerate(((24, 70, 5), (7, 37, 3))):
        print(f"case static layer {dt} call {call}: rows={rows} n={n}", flush=True)
        x, live, table, gs, ge = _inputs(rows, n, per_group, seed=10 + call)
        need = chronos2.layer_workspace_bytes(rows, n, D, HEADS * DH, DFF, code)
        assert 0 < need <= chronos2.LAYER_STATIC_BYTES
        ws = torch.empty(need // 4 + 64, dtype=torch.float32, device=DEV)
        x_ws, x_own, x_st = x.clone(), x.clone(), x.clone()
        chronos2.layer(x_ws, w, live, table, gs, ge, ws, rows, n, D, HEADS, DH, DFF, 1e-6, code)
        monkeypatch.setenv("JITCAST_HIP_GEMM", "own")
        chronos2.layer(x_own, w, live, table, gs, ge, ws, rows, n, D, HEADS, DH, DFF, 1e-6, code)
        monkeypatch.delenv("JITCAST_HIP_GEMM")
        chronos2.layer_static(x_st, w, live, table, gs, ge, rows, n, D, HEADS, DH, DFF, 1e-6, code)
        torch.cuda.synchronize()
        assert torch.isfinite(x_st).all()
        assert not torch.equal(x_st, x)  # the layer did run
        assert torch.equal(x_st, x_own)
        err = _rel(x_st, x_ws)
        print(f"  static vs workspace layer on hipBLASLt: rel err {err:.2e}", flush=True)
        assert err <= (2e-2 if dt == "bf16" else 1e-4)


def test_static_layer_rejects_past_its_scratch(gpu):
    """A request whose workspace exceeds the scratch fails on the host, naming the limit."""
    w = _weights(chronos2._lib.JC_F32)
    rows, n = 128, 133
    need = chronos2.layer_workspace_bytes(rows, n, D, HEADS * DH, DFF)
    assert need > chronos2.LAYER_STATIC_BYTES
    x = torch.zeros(rows * n, D, device=DEV)
    with pytest.raises(JitcastArgumentError, match="static scratch"):
        chronos2.layer_static(x, w, None, None, None, None, rows, n, D, HEADS, DH, DFF, 1e-6)
