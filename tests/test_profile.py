"""-Dchronos2.hip.profile / -Dtimestral.hip.profile: the per-kernel timing of jc_profile and
jc_profile_report (the counterpart of the reference's TornadoVM console profiler,
J/chronos2/tornado/Chronos2Forward.java:301-303). CPU: argument and state errors; GPU: a profiled
eager forward prints one line per kernel kind with the launch counts the forward makes."""
import ctypes

import numpy as np
import pytest

from jitcast_amd import _lib


def test_profile_null_context_is_an_error():
    assert _lib.lib().jc_profile(None, 1) == _lib.JC_EINVAL
    buf = ctypes.create_string_buffer(64)
    assert _lib.lib().jc_profile_report(None, buf, 64) == _lib.JC_EINVAL


def test_profile_option_is_strict():
    from jitcast_amd import options

    options.set_property("chronos2.hip.profile", "maybe")
    try:
        with pytest.raises(ValueError, match="chronos2.hip.profile"):
            options.boolean("chronos2.hip.profile", False)
    finally:
        options.set_property("chronos2.hip.profile", None)


@pytest.mark.gpu
def test_profiled_forward_reports_each_kernel(gpu, capfd):
    import torch

    from jitcast_amd import chronos2_model as cm
    from jitcast_amd import options, runtime
    from tests.test_gpu_forward import SMALL
    from tests.test_oracle_forward import _context

    ctx = runtime.context(0)
    buf = ctypes.create_string_buffer(256)
    assert _lib.lib().jc_profile_report(ctx.handle, buf, 256) == _lib.JC_ESTATE  # off
    options.set_property("chronos2.hip.profile", "true")
    try:
        m = cm.HipChronos2Model(SMALL, cm.random_weights(SMALL, seed=1, std=0.1))
        lay = cm.layout(SMALL, _context(2, 4, 200, lead_nan=[0, 40, 0, 17]), [0, 0, 1, 1], None, h=2)
        tok, _, _ = cm.prep(SMALL, lay)
        gs, ge = cm.chronos2.group_bounds(lay.group)
        dev = m.dev
        up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        m.forward_raw(up(tok), up(lay.live.reshape(-1)), up(gs), up(ge), lay.rows, lay.nc, lay.h)
        torch.cuda.synchronize()
    finally:
        options.set_property("chronos2.hip.profile", None)
    err = capfd.readouterr().err
    print(err)
    assert "chronos2.hip.profile forward rows=4" in err
    lines = {ln.split()[0] + " " + ln.split()[1]: ln.split() for ln in err.splitlines() if ln.startswith("c2 ")}
    layers = SMALL.num_layers
    assert int(lines["c2 time_attention_f32"][2]) == layers
    assert int(lines["c2 group_attention_f32"][2]) == layers
    assert "all timed launches" in err
    # profiling is off again afterwards
    assert _lib.lib().jc_profile_report(runtime.context(0).handle, buf, 256) == _lib.JC_ESTATE
