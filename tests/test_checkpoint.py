"""Checkpoint files and options on the CPU: the safetensors reader (SafeTensorsTest.java), the strict
config.json parse (Chronos2Config.fromJson), binding every tensor once with its exact shape
(Chronos2Weights.load), the write/load round trip the benchmark's synthetic checkpoints rely on, and
the strict -D option readers (J/util/Options.java)."""
import json
import struct

import numpy as np
import pytest

from jitcast_amd import checkpoint as ck
from jitcast_amd import options as opts
from jitcast_amd.chronos2_model import Chronos2Config, random_weights

SMALL = Chronos2Config(d_model=32, d_kv=8, d_ff=48, num_layers=2, num_heads=4, context_length=256, patch_size=16,
                       max_output_patches=4, quantiles=(0.1, 0.5, 0.9), time_encoding_scale=256)


def _write_raw(path, header: str, data):
    h = header.encode("utf-8")
    with open(path, "wb") as f:
        f.write(struct.pack("<q", len(h)) + h + np.asarray(data, "<f4").tobytes())


def test_reads_tensors_and_metadata(tmp_path):
    # an odd header length, so the data section starts unaligned (SafeTensorsTest.readsTensorsAndMetadata)
    header = ('{"__metadata__":{"k":"v"},"a":{"dtype":"F32","shape":[2,3],"data_offsets":[0,24]},'
              '"b":{"dtype":"F32","shape":[2],"data_offsets":[24,32]}}   ')
    _write_raw(tmp_path / "t.safetensors", header, [1, 2, 3, 4, 5, 6, -1.5, 7.25])
    with ck.SafeTensors(tmp_path / "t.safetensors") as st:
        assert st.metadata == {"k": "v"}
        assert len(st.tensors) == 2
        a = st.get("a").require_f32(2, 3)
        np.testing.assert_array_equal(a.to_numpy(), [[1, 2, 3], [4, 5, 6]])
        assert st.get("b").to_numpy()[1] == np.float32(7.25)


def test_rejects_shape_and_range_mismatch(tmp_path):
    _write_raw(tmp_path / "bad.safetensors", '{"a":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}', [1, 2])
    with pytest.raises(ValueError):
        ck.SafeTensors(tmp_path / "bad.safetensors")
    _write_raw(tmp_path / "ok.safetensors", '{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', [1, 2])
    with ck.SafeTensors(tmp_path / "ok.safetensors") as st:
        with pytest.raises(ValueError):
            st.get("a").require_f32(1, 2)
    with open(tmp_path / "short.safetensors", "wb") as f:
        f.write(struct.pack("<q", 1000) + b"{}")
    with pytest.raises(OSError):
        ck.SafeTensors(tmp_path / "short.safetensors")


def test_config_round_trip_and_defaults():
    c = ck.parse_config(ck.config_json(SMALL))
    assert c == SMALL
    doc = {"chronos_config": {"context_length": 64, "input_patch_size": 16, "input_patch_stride": 16,
                              "output_patch_size": 16, "quantiles": [0.25, 0.5, 0.75]}}
    c = ck.parse_config(json.dumps(doc))
    assert (c.d_model, c.d_kv, c.d_ff, c.num_layers, c.num_heads) == (512, 64, 2048, 6, 8)
    assert (c.max_output_patches, c.use_reg_token, c.use_arcsinh, c.time_encoding_scale) == (1, False, False, 64)


@pytest.mark.parametrize("edit,match", [
    (lambda d: d.update(unknown=1), "unknown config key"),
    (lambda d: d["chronos_config"].update(extra=1), "unknown config key"),
    (lambda d: d.pop("chronos_config"), "no chronos_config"),
    (lambda d: d.update(architectures=["T5Model"]), "not a Chronos-2"),
    (lambda d: d.update(is_gated_act=True), "ReLU"),
    (lambda d: d.update(dense_act_fn="gelu"), "ReLU"),
    (lambda d: d.update(torch_dtype="bfloat16"), "float32"),
    (lambda d: d["chronos_config"].update(output_patch_size=8), "patch"),
    (lambda d: d.update(d_kv=7), "even"),
    (lambda d: d["chronos_config"].update(quantiles=[0.5, 0.1]), "increasing"),
    (lambda d: d["chronos_config"].update(context_length=8), "hold a patch"),
])
def test_config_rejects(edit, match):
    d = json.loads(ck.config_json(SMALL))
    edit(d)
    with pytest.raises(ValueError, match=match):
        ck.parse_config(json.dumps(d))


def test_checkpoint_round_trip(tmp_path):
    w = random_weights(SMALL, seed=4)
    ck.write_chronos2(tmp_path, SMALL, w)
    c, got = ck.load_chronos2(tmp_path)
    assert c == SMALL
    assert sorted(k for k in got if k != "layers") == sorted(k for k in w if k != "layers")
    for k in w:
        if k != "layers":
            np.testing.assert_array_equal(got[k], w[k])
    for lg, lw in zip(got["layers"], w["layers"]):
        assert sorted(lg) == sorted(lw)
        for k in lw:
            np.testing.assert_array_equal(lg[k], lw[k])


def _rewrite(tmp_path, mutate):
    w = random_weights(SMALL, seed=4)
    ck.write_chronos2(tmp_path, SMALL, w)
    with ck.SafeTensors(tmp_path / "model.safetensors") as st:
        tensors = {n: st.get(n).to_numpy() for n in st.tensors}
    mutate(tensors)
    ck.write_safetensors(tmp_path / "model.safetensors", tensors)


def test_load_requires_every_tensor_once_with_its_shape(tmp_path):
    _rewrite(tmp_path, lambda t: t.update(extra=np.zeros(3, np.float32)))
    with pytest.raises(ValueError, match="unexpected tensors"):
        ck.load_chronos2(tmp_path)
    _rewrite(tmp_path, lambda t: t.pop("encoder.block.1.layer.2.mlp.wo.weight"))
    with pytest.raises(ValueError, match="no tensor"):
        ck.load_chronos2(tmp_path)
    _rewrite(tmp_path, lambda t: t.update({"encoder.final_layer_norm.weight": np.ones(31, np.float32)}))
    with pytest.raises(ValueError, match="expected F32"):
        ck.load_chronos2(tmp_path)


def test_options_are_strict(monkeypatch):
    monkeypatch.setenv("JITCAST_OPTS", "-Dchronos2.maxTokens=4096 -Dchronos2.hip.dtype=BF16 -Dx.bad=12z")
    assert opts.number("chronos2.maxTokens", 1, 1) == 4096
    assert opts.choice("chronos2.hip.dtype", "f32", "f32", "bf16", "fp16") == "bf16"
    with pytest.raises(ValueError, match=r"-Dx.bad=12z: expected a whole number"):
        opts.number("x.bad", 1, 1)
    assert opts.integer("unset.key", 7, 0) == 7
    opts.set_property("chronos2.maxTokens", "0")
    try:
        with pytest.raises(ValueError, match="at least 1"):
            opts.number("chronos2.maxTokens", 1, 1)
    finally:
        opts.set_property("chronos2.maxTokens", None)
    assert [opts.parse_bytes(s) for s in ("512MB", "8gb", " 3 KB", "12", "1.5GB", "x")] == [
        512 << 20, 8 << 30, 3 << 10, 12, -1, -1]
    opts.set_property("b", "maybe")
    try:
        with pytest.raises(ValueError, match="true or false"):
            opts.boolean("b", False)
    finally:
        opts.set_property("b", None)
