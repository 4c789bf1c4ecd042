"""Plans on the GPU: the attention entry points captured into one hipGraph per shape, replayed with
fresh inputs uploaded between replays (and eager work in between), every replay checked against
the eager result bit for bit; capture-state errors; adopted buffers."""
import ctypes

import numpy as np
import pytest
import torch

from jitcast_amd import JitcastError, _lib, chronos2, plans, timestral
from jitcast_amd.runtime import context
from tests import cases

pytestmark = pytest.mark.gpu


def _stage_inputs(seed, rows, n, heads, dh, inner):
    qkv = torch.from_numpy(cases.qkv(seed, rows * n, inner)).cuda()
    live = torch.from_numpy(cases.left_pad_live(seed, rows, n, n // 3).reshape(-1)).cuda()
    return qkv, live


def test_captured_plan_replays_match_eager(gpu):
    rows, n, heads, dh, inner = 24, 70, 2, 64, 128
    enc, ll = n - 4, n - 4
    group = cases.group_sizes(3, rows, 1, 6)
    gs, ge = (torch.from_numpy(x).cuda() for x in chronos2.group_bounds(group))
    table = torch.from_numpy(chronos2.rope_table(n, dh)).cuda()
    kv, known, position = cases.ts_layout(3, rows, enc, ll, n - enc, 0.3)
    kv_t = torch.from_numpy(kv.reshape(-1)).cuda()
    known_t = torch.from_numpy(known).cuda()
    pos_t = torch.from_numpy((position + enc).reshape(-1).astype(np.int32)).cuda()
    ts_table = torch.from_numpy(timestral.rope_table(enc, n, dh, 32)).cuda()
    qkv, live = _stage_inputs(1, rows, n, heads, dh, inner)
    gate = torch.from_numpy(cases.qkv(2, rows * n, inner)[:, :inner].copy()).cuda()
    outs = [torch.zeros(rows * n, inner, device="cuda") for _ in range(3)]

    def stage(o):
        chronos2.time_attention(qkv, o[0], live, rows, n, heads, dh, inner, table)
        chronos2.group_attention(qkv, o[1], live, gs, ge, rows, n, heads, dh, inner)
        timestral.time_attention(qkv, o[2], kv_t, known_t, pos_t, ts_table, gate, rows, enc, ll, n, heads, dh, inner)

    side = torch.cuda.Stream()  # default priority
    with torch.cuda.stream(side):
        with plans.capture(shape_key=rows * 100000 + n) as box:
            stage(outs)
    plan = box[0]
    assert plan.key == rows * 100000 + n
    try:
        for replay in range(3):
            fresh_qkv, fresh_live = _stage_inputs(10 + replay, rows, n, heads, dh, inner)
            with torch.cuda.stream(side):
                qkv.copy_(fresh_qkv)
                live.copy_(fresh_live)
                for o in outs:
                    o.fill_(float("nan"))
                plan.launch()
            side.synchronize()
            expect = [torch.zeros_like(o) for o in outs]
            stage(expect)  # eager, on the default stream
            torch.cuda.synchronize()
            for got, exp in zip(outs, expect):
                assert torch.equal(got, exp), f"replay {replay} differs from eager"
            torch.cuda.synchronize()
    finally:
        plan.close()


def test_capture_state_errors(gpu):
    ctx = context(0)
    h = ctypes.c_void_p()
    assert _lib.lib().jc_plan_end(ctx.handle, ctypes.byref(h)) == _lib.JC_ESTATE
    side = torch.cuda.Stream()
    buf = np.zeros(4, np.float32)
    dev = torch.zeros(4, device="cuda")
    with torch.cuda.stream(side):
        ctx = context(0)
        _lib.call("jc_plan_begin", ctx.handle, ctypes.c_uint64(7))
        assert _lib.lib().jc_plan_begin(ctx.handle, ctypes.c_uint64(8)) == _lib.JC_ESTATE
        rc = _lib.lib().jc_memcpy_h2d(ctx.handle, ctypes.c_void_p(dev.data_ptr()),
                                      buf.ctypes.data_as(ctypes.c_void_p), 16)
        assert rc == _lib.JC_ESTATE and "cannot be captured" in _lib.last_error()
        assert _lib.lib().jc_sync(ctx.handle) == _lib.JC_ESTATE
        _lib.call("jc_plan_end", ctx.handle, ctypes.byref(h))
    plan = plans.Plan(h)
    plan.launch()  # an empty graph replays
    side.synchronize()
    plan.close()
    plan.close()  # idempotent


def test_adopted_buffers_are_the_plan_footprint(gpu):
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        ctx = context(0)
        with plans.capture(shape_key=1) as box:
            pass
    plan = box[0]
    ptrs = []
    for nbytes in (1 << 20, 3 << 20):
        p = ctypes.c_void_p()
        _lib.call("jc_alloc", ctx.handle, nbytes, ctypes.byref(p))
        plan.adopt(p.value, nbytes)
        ptrs.append(p)
    assert plan.device_bytes() == 4 << 20
    plan.close()  # frees both buffers
    assert plan.device_bytes() == 0


def test_null_stream_cannot_be_captured(gpu):
    ctx = context(0)
    own = _lib.lib().jc_stream(ctx.handle)
    _lib.call("jc_set_stream", ctx.handle, None)
    try:
        with pytest.raises(JitcastError, match="null stream"):
            _lib.call("jc_plan_begin", ctx.handle, ctypes.c_uint64(1))
    finally:
        _lib.call("jc_set_stream", ctx.handle, ctypes.c_void_p(own))
