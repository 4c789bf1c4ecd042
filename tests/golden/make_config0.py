"""Writes tests/golden/config0.npz: config 0 (the Chronos-2 28M-class model, d_model 512, 8 x 64 heads,
6 layers, patch 16, 21 quantiles; random-init weights N(0, 0.02) from the portable RNG, seed 0,
RMSNorm weights 1, biases 0) run through the oracle: Chronos2Pipeline over CpuChronos2.forward, on
4 univariate series of 512 steps (sines of periods 24 and 168 with amplitudes U(0.5, 2), a linear
trend of slope U(-0.01, 0.01), N(0, 0.1) noise), horizon 64.

Stored: the inputs [4, 512], the quantiles [4, 21, 64], and the encoder's output after each layer
[6, 4 * 37, 512] of the one forward call (37 tokens per series: 32 context patches, [REG], 4 future
patches). Usage: python tests/golden/make_config0.py (a few seconds)."""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from jitcast_amd import synthetic  # noqa: E402
from jitcast_amd.chronos2_model import Chronos2Config  # noqa: E402
from oracle import c2_pipeline, oracle  # noqa: E402

CONFIG0 = Chronos2Config(d_model=512, d_kv=64, d_ff=2048, num_layers=6, num_heads=8)
HORIZON = 64
OUT = Path(__file__).resolve().parent / "config0.npz"


def run(w, series):
    layers = {}

    def fwd(context, group, future, op):
        sink = (lambda name, x: layers.setdefault(name, np.array(x, np.float32))) if not layers else None
        return oracle.c2_model_forward(CONFIG0, w, np.asarray(context, np.float32), np.asarray(group, np.int32),
                                       np.asarray(future, np.float32), op, sink=sink)

    q = c2_pipeline.forecast(CONFIG0, fwd, [([row], None, None) for row in series], HORIZON)
    return np.stack([v[0] for v in q]), np.stack([layers[f"layer{i}"] for i in range(CONFIG0.num_layers)])


def main():
    w = synthetic.c2_portable_weights(CONFIG0, seed=0)
    series = synthetic.c2_config0_series()
    quantiles, layers = run(w, series)
    np.savez_compressed(OUT, inputs=series, quantiles=quantiles, layers=layers)
    print(f"wrote {OUT}: quantiles {quantiles.shape}, layers {layers.shape}")


if __name__ == "__main__":
    main()
