"""Chronos-2 checkpoints on disk: config.json and model.safetensors, read as strictly as the reference
reads them, and written for the benchmark's random-init configurations.

  parse_config        Chronos2Config.fromJson (J/chronos2/Chronos2Config.java:64-69, 118-191): only
                      known keys, the ReLU feed-forward layer, float32 weights, equal patch sizes
  SafeTensors         a read-only memory-mapped safetensors file (J/io/SafeTensors.java:40-150):
                      8-byte little-endian header length, JSON header, tensor bytes; each tensor's byte
                      range must match its dtype and shape
  Tensor.require_f32  the exact-shape F32 check of Tensor.requireF32 (J/io/Tensor.java)
  load_chronos2       Chronos2Weights.load (J/chronos2/Chronos2Weights.java:77-100, 158-201): every
                      tensor bound exactly once by name and shape, extra tensors rejected; returns the
                      config and the weights in the layout HipChronos2Model takes (q|k|v fused per
                      attention sublayer, Chronos2Weights.qkv)
  write_safetensors, write_chronos2
                      the inverse, for synthetic checkpoints
  parse_ts_config     TimestralConfig.fromJson (J/timestral/TimestralConfig.java:162-240): only known
                      keys, no biases in attention or MLP, no global stabilisation, the block schedule,
                      increasing quantile knots holding 0.5, the attention gates
  load_timestral      TimestralWeights.load (J/timestral/TimestralWeights.java:83-120): every tensor
                      bound once by name and exact F32 shape; the weights come back in
                      HipTimestralModel's layout (q|k|v rows heads-major, TimestralWeights.qkv; the
                      MLP up projection with its SiLU half first, TimestralWeights.mlpUp)
  write_timestral     the inverse, for synthetic checkpoints

Errors are ValueError (the reference's IllegalArgumentException) or OSError.
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

_DTYPES = {"F32": ("<f4", 4), "F16": ("<f2", 2), "BF16": (None, 2), "F64": ("<f8", 8), "I64": ("<i8", 8),
           "I32": ("<i4", 4), "U8": ("u1", 1), "BOOL": ("?", 1)}

_KEYS = {"architectures", "chronos_config", "chronos_pipeline_class", "d_ff", "d_kv", "d_model", "dense_act_fn",
         "dropout_rate", "feed_forward_proj", "initializer_factor", "is_gated_act", "layer_norm_epsilon", "model_type",
         "num_heads", "num_layers", "pad_token_id", "reg_token_id", "rope_theta", "torch_dtype", "dtype",
         "transformers_version", "use_cache", "vocab_size", "attn_implementation"}
_CHRONOS_KEYS = {"context_length", "input_patch_size", "input_patch_stride", "output_patch_size", "max_output_patches",
                 "quantiles", "use_reg_token", "use_arcsinh", "time_encoding_scale"}


def _reject_constant(name):
    raise ValueError(f"not JSON: {name}")


def _parse_object(text: str) -> dict:
    try:
        v = json.loads(text, parse_constant=_reject_constant)
    except json.JSONDecodeError as e:
        raise ValueError(f"bad JSON: {e}") from None
    if not isinstance(v, dict):
        raise ValueError("Expected a JSON object")
    return v


def _is_num(v) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def _str(m: dict, k: str, default: str) -> str:
    v = m.get(k)
    return v if isinstance(v, str) else default


def _num(m: dict, k: str, default: float) -> float:
    v = m.get(k)
    return float(v) if _is_num(v) else default


def _int(m: dict, k: str, default: int) -> int:
    v = m.get(k)
    return int(v) if _is_num(v) else default  # Number.intValue truncates toward zero


def _bool(m: dict, k: str, default: bool) -> bool:
    v = m.get(k)
    return v if isinstance(v, bool) else default


def _require_known(m: dict, keys: set) -> None:
    for k in m:
        if k not in keys:
            raise ValueError(f"unknown config key: {k}")


def parse_config(text: str):
    """A Chronos2Config from a config.json document (Chronos2Config.fromJson)."""
    from .chronos2_model import Chronos2Config

    c = _parse_object(text)
    _require_known(c, _KEYS)
    cc = c.get("chronos_config")
    if cc is None:
        raise ValueError("not a Chronos-2 config: no chronos_config")
    if not isinstance(cc, dict):
        raise ValueError("chronos_config must be an object")
    _require_known(cc, _CHRONOS_KEYS)
    arch = c.get("architectures")
    if isinstance(arch, list) and "Chronos2Model" not in arch:
        raise ValueError(f"not a Chronos-2 checkpoint: {arch}")
    act = _str(c, "dense_act_fn", _str(c, "feed_forward_proj", "relu"))
    if act != "relu" or _bool(c, "is_gated_act", False) or _str(c, "feed_forward_proj", "relu") != "relu":
        raise ValueError(f"only the ReLU feed-forward layer is supported, got {act}")
    dtype = _str(c, "torch_dtype", _str(c, "dtype", "float32"))
    if dtype != "float32":
        raise ValueError(f"only float32 checkpoints are supported, got {dtype}")
    patch = _int(cc, "input_patch_size", 0)
    if patch != _int(cc, "output_patch_size", 0) or patch != _int(cc, "input_patch_stride", 0):
        raise ValueError("input and output patch sizes and the patch stride must be equal")
    qs = cc.get("quantiles")
    if not isinstance(qs, list) or not all(_is_num(q) for q in qs):
        raise ValueError("chronos_config.quantiles must be a list of numbers")
    context = _int(cc, "context_length", 0)
    f32 = lambda v: float(np.float32(v))  # noqa: E731  (the reference keeps these as float)
    cfg = Chronos2Config(
        d_model=_int(c, "d_model", 512), d_kv=_int(c, "d_kv", 64), d_ff=_int(c, "d_ff", 2048),
        num_layers=_int(c, "num_layers", 6), num_heads=_int(c, "num_heads", 8),
        layer_norm_eps=f32(_num(c, "layer_norm_epsilon", 1e-6)), rope_theta=f32(_num(c, "rope_theta", 10000.0)),
        context_length=context, patch_size=patch, max_output_patches=_int(cc, "max_output_patches", 1),
        quantiles=tuple(float(q) for q in qs), use_reg_token=_bool(cc, "use_reg_token", False),
        use_arcsinh=_bool(cc, "use_arcsinh", False), time_encoding_scale=_int(cc, "time_encoding_scale", context))
    _validate(cfg)
    return cfg


def _validate(c) -> None:
    """Chronos2Config.validate (Chronos2Config.java:168-183)."""
    if min(c.d_model, c.d_kv, c.d_ff, c.num_layers, c.num_heads, c.patch_size, c.max_output_patches) < 1:
        raise ValueError("non-positive model dimensions")
    if c.d_kv % 2:
        raise ValueError(f"d_kv must be even for RoPE, got {c.d_kv}")
    if c.context_length < c.patch_size or c.time_encoding_scale < 1:
        raise ValueError("context_length must hold a patch")
    for i, q in enumerate(c.quantiles):
        if not (0 < q < 1) or (i > 0 and not c.quantiles[i - 1] < q):
            raise ValueError("quantiles must be increasing and in (0, 1)")


def config_json(c) -> str:
    """The config.json document of a Chronos2Config, with the keys Amazon's checkpoints carry."""
    doc = {
        "architectures": ["Chronos2Model"], "model_type": "t5", "torch_dtype": "float32",
        "d_model": c.d_model, "d_kv": c.d_kv, "d_ff": c.d_ff, "num_layers": c.num_layers, "num_heads": c.num_heads,
        "layer_norm_epsilon": c.layer_norm_eps, "rope_theta": c.rope_theta, "dense_act_fn": "relu",
        "feed_forward_proj": "relu", "is_gated_act": False, "vocab_size": c.vocab_size,
        "chronos_config": {
            "context_length": c.context_length, "input_patch_size": c.patch_size, "input_patch_stride": c.patch_size,
            "output_patch_size": c.patch_size, "max_output_patches": c.max_output_patches,
            "quantiles": list(c.quantiles), "use_reg_token": c.use_reg_token, "use_arcsinh": c.use_arcsinh,
            "time_encoding_scale": c.time_encoding_scale,
        },
    }
    return json.dumps(doc, indent=2)


@dataclass(frozen=True)
class Tensor:
    name: str
    dtype: str
    shape: tuple
    data: np.ndarray  # the tensor's bytes (uint8 view of the mapping)

    def elements(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    def require_f32(self, *expected) -> "Tensor":
        """Fails unless the tensor is F32 with exactly `expected` as its shape."""
        if self.dtype != "F32" or tuple(self.shape) != tuple(int(e) for e in expected):
            raise ValueError(f"{self.name}: expected F32{list(expected)}, found {self.dtype}{list(self.shape)}")
        return self

    def to_numpy(self) -> np.ndarray:
        """A writable float32 copy of an F32 tensor."""
        if self.dtype != "F32":
            raise RuntimeError(f"{self.name} is {self.dtype}, not F32")
        return np.frombuffer(self.data.tobytes(), dtype="<f4").astype(np.float32).reshape(self.shape)


class SafeTensors:
    """A memory-mapped safetensors file; tensors are views of one mapping, kept until close()."""

    def __init__(self, path):
        path = Path(path)
        self._mm = np.memmap(path, dtype=np.uint8, mode="r")
        size = self._mm.size
        if size < 8:
            raise OSError(f"{path}: bad safetensors header length (file of {size} bytes)")
        (hlen,) = struct.unpack("<q", self._mm[:8].tobytes())
        if hlen <= 0 or 8 + hlen > size:
            raise OSError(f"{path}: bad safetensors header length {hlen}")
        header = _parse_object(self._mm[8: 8 + hlen].tobytes().decode("utf-8"))
        data = self._mm[8 + hlen:]
        self.tensors: dict = {}
        self.metadata: dict = {}
        for name, info in header.items():
            if name == "__metadata__":
                self.metadata = {str(k): v if isinstance(v, str) else json.dumps(v) for k, v in info.items()}
                continue
            self.tensors[name] = self._tensor(name, info, data)

    @staticmethod
    def _tensor(name: str, info: dict, data: np.ndarray) -> Tensor:
        dt = info.get("dtype")
        if dt not in _DTYPES:
            raise ValueError(f"{name}: unknown dtype {dt}")
        shape = tuple(int(s) for s in info.get("shape", []))
        elements = int(np.prod(shape, dtype=np.int64)) if shape else 1
        begin, end = (int(o) for o in info.get("data_offsets", [0, -1]))
        if end - begin != elements * _DTYPES[dt][1]:
            raise ValueError(f"{name}: byte range {end - begin} does not match shape {list(shape)} of {dt}")
        if begin < 0 or end > data.size:
            raise ValueError(f"{name}: byte range [{begin}, {end}) outside the data section of {data.size} bytes")
        return Tensor(name, dt, shape, data[begin:end])

    def get(self, name: str) -> Tensor:
        t = self.tensors.get(name)
        if t is None:
            raise ValueError(f"no tensor '{name}'")
        return t

    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def close(self) -> None:
        self.tensors = {}
        mm, self._mm = self._mm, None
        if mm is not None:
            del mm

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False


def write_safetensors(path, tensors: dict, metadata: dict | None = None) -> None:
    """Writes float32 arrays as F32 tensors, in the given order, the header padded to 8 bytes."""
    header, offset = {}, 0
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    arrays = []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a, dtype="<f4")
        header[name] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [offset, offset + a.nbytes]}
        offset += a.nbytes
        arrays.append(a)
    raw = json.dumps(header, separators=(",", ":")).encode("utf-8")
    raw += b" " * (-len(raw) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<q", len(raw)))
        f.write(raw)
        for a in arrays:
            f.write(a.tobytes())


# ---- Chronos-2 weights: names and shapes of Chronos2Weights.load --------------------------------

def _chronos2_names(c) -> list:
    """(name, shape, key) of every tensor a Chronos-2 checkpoint holds, in binding order; key says
    where HipChronos2Model's weight dict keeps it."""
    d, inner, ff, p, q = c.d_model, c.inner, c.d_ff, c.patch_size, c.num_quantiles
    out = [("shared.weight", (c.vocab_size, d), "shared")]

    def residual(prefix, key, din, hidden, dout):
        for part, short, shp in (("hidden_layer", "hidden", (hidden, din)), ("output_layer", "output", (dout, hidden)),
                                 ("residual_layer", "residual", (dout, din))):
            out.append((f"{prefix}.{part}.weight", shp, f"{key}_{short}_w"))
            out.append((f"{prefix}.{part}.bias", (shp[0],), f"{key}_{short}_b"))

    residual("input_patch_embedding", "in", 3 * p, ff, d)
    for i in range(c.num_layers):
        s = f"encoder.block.{i}.layer."
        for sub, kind in (("0", "time"), ("1", "group")):
            a = s + sub + ".self_attention."
            out.append((s + sub + ".layer_norm.weight", (d,), (i, f"{kind}_norm")))
            for proj in ("q", "k", "v"):
                out.append((a + proj + ".weight", (inner, d), (i, f"{kind}_{proj}")))
            out.append((a + "o.weight", (d, inner), (i, f"{kind}_o")))
        out.append((s + "2.layer_norm.weight", (d,), (i, "mlp_norm")))
        out.append((s + "2.mlp.wi.weight", (ff, d), (i, "wi")))
        out.append((s + "2.mlp.wo.weight", (d, ff), (i, "wo")))
    out.append(("encoder.final_layer_norm.weight", (d,), "final_norm"))
    residual("output_patch_embedding", "out", d, ff, q * p)
    return out


def load_chronos2(checkpoint_dir) -> tuple:
    """Chronos2Weights.load: (Chronos2Config, weights) from <dir>/config.json and
    <dir>/model.safetensors. Every tensor is bound once with its exact F32 shape; a missing tensor,
    a wrong shape or an unexpected extra tensor fails the load."""
    d = Path(checkpoint_dir)
    from .chronos2_model import Chronos2Config

    c = Chronos2Config.load(d / "config.json")
    with SafeTensors(d / "model.safetensors") as st:
        bound: set = set()
        w: dict = {"layers": [dict() for _ in range(c.num_layers)]}
        for name, shape, key in _chronos2_names(c):
            if name in bound:
                raise RuntimeError(f"{name} bound twice")
            bound.add(name)
            if name not in st:
                raise ValueError(f"checkpoint has no tensor {name}")
            arr = st.get(name).require_f32(*shape).to_numpy()
            if isinstance(key, tuple):
                w["layers"][key[0]][key[1]] = arr
            else:
                w[key] = arr
        unbound = sorted(set(st.tensors) - bound)
        if unbound:
            raise ValueError(f"unexpected tensors in checkpoint: {unbound}")
    for lw in w["layers"]:  # the fused q|k|v of each attention sublayer (Chronos2Weights.qkv)
        for kind in ("time", "group"):
            lw[f"{kind}_qkv"] = np.concatenate([lw.pop(f"{kind}_q"), lw.pop(f"{kind}_k"), lw.pop(f"{kind}_v")])
    return c, w


def write_chronos2(checkpoint_dir, c, weights: dict) -> Path:
    """Writes config.json and model.safetensors for weights in HipChronos2Model's layout (the fused
    q|k|v split back into q, k and v)."""
    d = Path(checkpoint_dir)
    d.mkdir(parents=True, exist_ok=True)
    (d / "config.json").write_text(config_json(c), encoding="utf-8")
    inner = c.inner
    tensors = {}
    for name, _shape, key in _chronos2_names(c):
        if isinstance(key, tuple):
            lw = weights["layers"][key[0]]
            k = key[1]
            if k[-2:] in ("_q", "_k", "_v"):
                part = "qkv".index(k[-1])
                tensors[name] = lw[k[:-2] + "_qkv"][part * inner: (part + 1) * inner]
            else:
                tensors[name] = lw[k]
        else:
            tensors[name] = weights[key]
    write_safetensors(d / "model.safetensors", tensors, {"format": "pt"})
    return d


# ---- Timestral ---------------------------------------------------------------------------------

_TS_KEYS = {"patch_size", "d_model", "num_heads", "mlp_hidden_dim", "block_schedule", "quantile_knots", "block_size",
            "context_length", "rope_theta", "rope_partial_factor", "norm_eps", "attn_bias", "mlp_bias", "time_attn_gate",
            "variate_attn_gate", "minimum_scale", "use_asinh", "stabilize_with_global", "covariate_enabled",
            "split_context_horizon_attn", "attend_missing_patches", "quantile_width_factor"}
_TS_KINDS = {"time": (True,), "variate": (False,), "time_variate": (True, False), "variate_time": (False, True)}


def _ts_gate(m: dict, key: str) -> bool:
    g = _str(m, key, "sdpa_sigmoid")
    if g == "sdpa_sigmoid":
        return True
    if g == "none":
        return False
    raise ValueError(f"unknown attention gate {g}")


def parse_ts_config(text: str):
    """A TimestralConfig from a config.json document (TimestralConfig.fromJson)."""
    from .timestral_model import TimestralConfig

    c = _parse_object(text)
    _require_known(c, _TS_KEYS)
    for key in ("attn_bias", "mlp_bias", "stabilize_with_global"):
        if _bool(c, key, False):
            raise ValueError(f"{key} = true is not supported")
    sched = c.get("block_schedule")
    if not isinstance(sched, list):
        raise ValueError("block_schedule must be a list")
    layers = []
    for kind in sched:
        if kind not in _TS_KINDS:
            raise ValueError(f"unknown layer kind {kind}")
        layers.append(_TS_KINDS[kind])
    knots = c.get("quantile_knots")
    if not isinstance(knots, list) or not all(_is_num(q) for q in knots):
        raise ValueError("quantile_knots must be a list of numbers")
    f32 = lambda v: float(np.float32(v))  # noqa: E731  (the reference keeps these as float)
    cfg = TimestralConfig(
        patch_size=_int(c, "patch_size", 0), d_model=_int(c, "d_model", 0), num_heads=_int(c, "num_heads", 0),
        mlp_hidden_dim=_int(c, "mlp_hidden_dim", 0), layers=tuple(layers), quantiles=tuple(float(q) for q in knots),
        rope_theta=f32(_num(c, "rope_theta", 10000.0)), rope_partial_factor=f32(_num(c, "rope_partial_factor", 0.5)),
        norm_eps=f32(_num(c, "norm_eps", 1e-6)), time_attn_gate=_ts_gate(c, "time_attn_gate"),
        variate_attn_gate=_ts_gate(c, "variate_attn_gate"), minimum_scale=f32(_num(c, "minimum_scale", 1e-6)),
        use_asinh=_bool(c, "use_asinh", True), quantile_width_factor=f32(_num(c, "quantile_width_factor", 2.0)),
        covariate_enabled=_bool(c, "covariate_enabled", True),
        attend_missing=_bool(c, "attend_missing_patches", True), block_size=_int(c, "block_size", 0),
        context_length=_int(c, "context_length", 0))
    _ts_validate(cfg)
    return cfg


def _ts_validate(c) -> None:
    """TimestralConfig.validate (TimestralConfig.java:211-227)."""
    if c.patch_size < 1 or c.d_model < 1 or c.num_heads < 1 or c.d_model % c.num_heads:
        raise ValueError(f"d_model {c.d_model} is not divisible by num_heads {c.num_heads}")
    if c.rope_dim <= 0 or c.rope_dim % 2:
        raise ValueError(f"rope_partial_factor {c.rope_partial_factor} gives rope_dim {c.rope_dim}")
    for i in range(1, len(c.quantiles)):
        if not c.quantiles[i - 1] < c.quantiles[i]:
            raise ValueError("quantile_knots must be increasing")
    if 0.5 not in c.quantiles:
        raise ValueError("no 0.5 quantile knot")
    if c.context_length % c.patch_size:
        raise ValueError("context_length must be a multiple of patch_size")


def ts_config_json(c) -> str:
    """The config.json document of a TimestralConfig."""
    kinds = {v: k for k, v in _TS_KINDS.items()}
    doc = {
        "patch_size": c.patch_size, "d_model": c.d_model, "num_heads": c.num_heads, "mlp_hidden_dim": c.mlp_hidden_dim,
        "block_schedule": [kinds[tuple(bool(x) for x in axes)] for axes in c.layers],
        "quantile_knots": list(c.quantiles), "block_size": c.block_size, "context_length": c.context_length,
        "rope_theta": c.rope_theta, "rope_partial_factor": c.rope_partial_factor, "norm_eps": c.norm_eps,
        "attn_bias": False, "mlp_bias": False, "time_attn_gate": "sdpa_sigmoid" if c.time_attn_gate else "none",
        "variate_attn_gate": "sdpa_sigmoid" if c.variate_attn_gate else "none", "minimum_scale": c.minimum_scale,
        "use_asinh": c.use_asinh, "covariate_enabled": c.covariate_enabled,
        "attend_missing_patches": c.attend_missing, "quantile_width_factor": c.quantile_width_factor,
    }
    return json.dumps(doc, indent=2)


def _timestral_names(c) -> list:
    """(name, shape, key) of every tensor a Timestral checkpoint holds, in binding order
    (TimestralWeights.java:92-117); key says where HipTimestralModel's weight dict keeps it."""
    d, p, f = c.d_model, c.patch_size, c.mlp_hidden_dim
    out = []

    def residual(prefix, key, din, hidden, dout, bias):
        for part, short, shp in (("hidden_layer", "hidden", (hidden, din)), ("output_layer", "output", (dout, hidden)),
                                 ("residual_layer", "residual", (dout, din))):
            out.append((f"{prefix}.{part}.weight", shp, f"{key}_{short}_w"))
            if bias:
                out.append((f"{prefix}.{part}.bias", (shp[0],), f"{key}_{short}_b"))

    residual("representation.patch_proj", "embed", 2 * p, 4 * d, d, True)
    out.append(("representation.forecast_query", (d,), "query"))
    for i, axes in enumerate(c.layers):
        s = f"transformer.layers.{i}"
        for a, time in enumerate(axes):
            gated = c.time_attn_gate if time else c.variate_attn_gate
            out.append((f"{s}.attn_norms.{a}.scale", (d,), (i, a, "norm")))
            out.append((f"{s}.attns.{a}.wQKV.weight", (3 * d, d), (i, a, "qkv")))
            if gated:
                out.append((f"{s}.attns.{a}._gate.weight", (d, d), (i, a, "gate")))
            out.append((f"{s}.attns.{a}.wO.weight", (d, d), (i, a, "wo")))
        out.append((f"{s}.mlp_norm.scale", (d,), (i, None, "mlp_norm")))
        out.append((f"{s}.mlp.w12.weight", (2 * f, d), (i, None, "up")))
        out.append((f"{s}.mlp.w3.weight", (d, f), (i, None, "down")))
    out.append(("transformer.out_norm.scale", (d,), "out_norm"))
    residual("head.projection", "head", d, 4 * d, p * c.num_quantiles, False)
    return out


def _qkv_heads_major(c, w: np.ndarray) -> np.ndarray:
    """TimestralWeights.qkv: checkpoint row s*d + e*heads + h to engine row s*d + h*dh + e."""
    d, heads, dh = c.d_model, c.num_heads, c.head_dim
    return np.ascontiguousarray(w.reshape(3, dh, heads, d).transpose(0, 2, 1, 3).reshape(3 * d, d))


def _qkv_checkpoint(c, w: np.ndarray) -> np.ndarray:
    d, heads, dh = c.d_model, c.num_heads, c.head_dim
    return np.ascontiguousarray(w.reshape(3, heads, dh, d).transpose(0, 2, 1, 3).reshape(3 * d, d))


def _swap_halves(w: np.ndarray) -> np.ndarray:
    """TimestralWeights.mlpUp: the two halves of w12 exchanged (its own inverse)."""
    f = w.shape[0] // 2
    return np.ascontiguousarray(np.concatenate([w[f:], w[:f]]))


def load_timestral(checkpoint_dir) -> tuple:
    """TimestralWeights.load: (TimestralConfig, weights) from <dir>/config.json and
    <dir>/model.safetensors, the weights in HipTimestralModel's layout (see random_weights)."""
    d = Path(checkpoint_dir)
    c = parse_ts_config((d / "config.json").read_text(encoding="utf-8"))
    with SafeTensors(d / "model.safetensors") as st:
        bound: set = set()
        w: dict = {"layers": [{"attentions": [{"time": bool(t), "gate": None} for t in axes]} for axes in c.layers]}
        for name, shape, key in _timestral_names(c):
            if name in bound:
                raise RuntimeError(f"{name} bound twice")
            bound.add(name)
            if name not in st:
                raise ValueError(f"checkpoint has no tensor {name}")
            arr = st.get(name).require_f32(*shape).to_numpy()
            if isinstance(key, tuple):
                layer, a, k = key
                if k == "qkv":
                    arr = _qkv_heads_major(c, arr)
                elif k == "up":
                    arr = _swap_halves(arr)
                (w["layers"][layer] if a is None else w["layers"][layer]["attentions"][a])[k] = arr
            else:
                w[key] = arr
        unbound = sorted(set(st.tensors) - bound)
        if unbound:
            raise ValueError(f"unexpected tensors in checkpoint: {unbound}")
    return c, w


def write_timestral(checkpoint_dir, c, weights: dict) -> Path:
    """Writes config.json and model.safetensors for weights in HipTimestralModel's layout."""
    d = Path(checkpoint_dir)
    d.mkdir(parents=True, exist_ok=True)
    (d / "config.json").write_text(ts_config_json(c), encoding="utf-8")
    tensors = {}
    for name, _shape, key in _timestral_names(c):
        if isinstance(key, tuple):
            layer, a, k = key
            arr = (weights["layers"][layer] if a is None else weights["layers"][layer]["attentions"][a])[k]
            if k == "qkv":
                arr = _qkv_checkpoint(c, np.asarray(arr, np.float32))
            elif k == "up":
                arr = _swap_halves(np.asarray(arr, np.float32))
        else:
            arr = weights[key]
        tensors[name] = np.ascontiguousarray(arr, np.float32)
    write_safetensors(d / "model.safetensors", tensors)
    return d
