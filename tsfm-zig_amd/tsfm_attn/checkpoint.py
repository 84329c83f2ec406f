"""Local checkpoints: the safetensors file format and the Chronos-Bolt checkpoint layout.

- :class:`Weights` reads a safetensors file the way src/core/safetensors.zig:32-97 does: an 8-byte
  little-endian header length, a JSON header of {name: {dtype, shape, data_offsets}}, then the
  data; F32 tensors are used in place (memory-mapped), F16 and BF16 are widened to float32 when
  first read; a missing name, another dtype or an element count other than the expected one is an
  error with the reference's message.
- :func:`write_safetensors` writes that format (F32, F16 or BF16).
- :func:`parse_bolt_config` parses and validates a Chronos-Bolt ``config.json``
  (src/chronos_bolt/config.zig:10-66): a T5 config plus its ``chronos_config`` block.
- :func:`load_bolt` reads ``config.json`` + ``model.safetensors`` under the tensor names of
  src/chronos_bolt/model.zig:101-160 and src/core/resblock.zig:24-55 into device tensors;
  :class:`BoltForecaster` forecasts any horizon with them through tsfm_bolt_forecast_horizon.
- :func:`write_bolt_checkpoint` writes such a directory from in-memory weights (for random-init
  checkpoints of a given shape).
"""
from __future__ import annotations

import json
import mmap
import os
from typing import Dict, Optional

import numpy as np

_DTYPES = {"F32": (np.float32, 4), "F16": (np.float16, 2), "BF16": (np.uint16, 2)}


class SafetensorsError(ValueError):
    """A checkpoint the reader refuses (the reference's error.InvalidSafetensors, MissingTensor,
    UnsupportedDtype, ShapeMismatch, MisalignedTensor)."""


class Weights:
    """A memory-mapped safetensors file (safetensors.zig Weights)."""

    def __init__(self, path: str):
        self.path = str(path)
        self._f = open(self.path, "rb")
        size = os.fstat(self._f.fileno()).st_size
        if size < 8:
            self._f.close()
            raise SafetensorsError(f"{self.path}: not a safetensors file (shorter than its header length)")
        self._map = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        hlen = int.from_bytes(self._map[:8], "little")
        if 8 + hlen > size:
            self.close()
            raise SafetensorsError(f"{self.path}: header length {hlen} runs past the end of the file")
        self.header = json.loads(bytes(self._map[8:8 + hlen]).decode("utf-8"))
        self.data_start = 8 + hlen

    def close(self) -> None:
        if getattr(self, "_map", None) is not None:
            try:
                self._map.close()
            except BufferError:
                pass  # F32 arrays still view the mapping: it is unmapped when the last of them goes
            self._map = None
        if getattr(self, "_f", None) is not None:
            self._f.close()
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def names(self):
        return [k for k in self.header if k != "__metadata__"]

    def get(self, name: str, numel: int) -> np.ndarray:
        """The named tensor as a flat float32 array of `numel` elements (Weights.get)."""
        entry = self.header.get(name)
        if entry is None or name == "__metadata__":
            raise SafetensorsError(f"missing tensor: {name}")
        dtype = entry["dtype"]
        if dtype not in _DTYPES:
            raise SafetensorsError(f"tensor {name} has unsupported dtype {dtype}")
        np_t, elem = _DTYPES[dtype]
        begin, end = (int(v) for v in entry["data_offsets"])
        if not 0 <= begin <= end or self.data_start + end > len(self._map):
            raise SafetensorsError(f"tensor {name}: data offsets {begin}..{end} outside the file")
        if end - begin != numel * elem:
            raise SafetensorsError(f"tensor {name}: expected {numel} elements, file has {(end - begin) // elem}")
        at = self.data_start + begin
        if elem == 4:
            if at % 4:
                raise SafetensorsError(f"tensor {name} is not 4-byte aligned in the file")
            return np.frombuffer(self._map, dtype=np.float32, count=numel, offset=at)
        raw = np.frombuffer(self._map, dtype=np.dtype(np_t).newbyteorder("<"), count=numel, offset=at)
        if dtype == "BF16":  # the high half of an f32
            return (raw.astype(np.uint32) << 16).view(np.float32)
        return raw.astype(np.float32)


def write_safetensors(path: str, tensors: Dict[str, np.ndarray], dtype: str = "F32",
                      metadata: Optional[Dict[str, str]] = None) -> None:
    """Write `tensors` (name -> array) as a safetensors file, every tensor as `dtype` (F32, F16 or
    BF16: BF16 rounds to nearest even). Tensors follow one another in name order; the header is
    padded with spaces to a multiple of 8 bytes, so F32 data stays 4-byte aligned."""
    if dtype not in _DTYPES:
        raise ValueError(f"dtype {dtype}: F32, F16 or BF16")
    blobs, header, off = [], {}, 0
    for name in sorted(tensors):
        a = np.asarray(tensors[name], np.float32)
        if dtype == "F32":
            b = a.astype("<f4").tobytes()
        elif dtype == "F16":
            b = a.astype("<f2").tobytes()
        else:
            u = np.ascontiguousarray(a).view(np.uint32).astype(np.uint64)
            r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype("<u2")
            b = r.tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    if metadata:
        header["__metadata__"] = dict(metadata)
    h = json.dumps(header, separators=(",", ":")).encode("utf-8")
    h += b" " * ((8 - (8 + len(h)) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


# ---- Chronos-Bolt -----------------------------------------------------------------------------

BOLT_ARCHITECTURE = "ChronosBoltModelForForecasting"


def parse_bolt_config(text: str) -> dict:
    """config.zig parse + validate: the fields the model reads, with their defaults; unknown fields
    ignored. Raises ValueError for what validate() refuses."""
    raw = json.loads(text)
    c = dict(layer_norm_epsilon=1e-6, dense_act_fn="relu", relative_attention_num_buckets=32,
             relative_attention_max_distance=128, decoder_start_token_id=0, reg_token_id=1)
    for k in ("d_model", "d_ff", "num_heads", "d_kv", "num_layers", "num_decoder_layers", "chronos_config"):
        if k not in raw:
            raise ValueError(f"config.json: missing field {k}")
    for k in list(c) + ["d_model", "d_ff", "num_heads", "d_kv", "num_layers", "num_decoder_layers"]:
        if k in raw:
            c[k] = raw[k]
    cc = raw["chronos_config"]
    for k in ("context_length", "input_patch_size", "input_patch_stride", "prediction_length", "quantiles"):
        if k not in cc:
            raise ValueError(f"config.json: missing chronos_config.{k}")
    c["chronos_config"] = dict(context_length=cc["context_length"], input_patch_size=cc["input_patch_size"],
                               input_patch_stride=cc["input_patch_stride"], prediction_length=cc["prediction_length"],
                               quantiles=[float(v) for v in cc["quantiles"]],
                               use_reg_token=bool(cc.get("use_reg_token", False)))
    x = c["chronos_config"]
    vocab = 2 if x["use_reg_token"] else 1
    if min(c["d_model"], c["d_ff"], c["num_heads"], c["d_kv"]) == 0 or c["num_layers"] == 0 or \
            c["num_decoder_layers"] == 0 or x["input_patch_size"] == 0 or x["prediction_length"] == 0 or \
            x["context_length"] == 0 or not x["quantiles"]:
        raise ValueError("InvalidConfig")
    if x["input_patch_stride"] != x["input_patch_size"]:
        raise ValueError("UnsupportedPatchStride: overlapping patches")
    if c["dense_act_fn"] != "relu":
        raise ValueError(f"UnsupportedActivation: {c['dense_act_fn']}")
    nb = c["relative_attention_num_buckets"]
    if nb < 4 or nb % 2:
        raise ValueError("InvalidConfig: relative_attention_num_buckets")
    if c["reg_token_id"] >= vocab or c["decoder_start_token_id"] >= vocab:
        raise ValueError("InvalidConfig: token ids")
    c["vocab"] = vocab
    return c


def bolt_config_dict(d_model: int, d_ff: int, num_heads: int, num_layers: int, num_decoder_layers: int,
                     context_length: int, patch: int, prediction_length: int, quantiles, eps: float = 1e-6,
                     buckets: int = 32, max_distance: int = 128) -> dict:
    """A Chronos-Bolt config.json body (T5 fields + chronos_config) with [REG] (token 1) and the
    decoder start token 0."""
    return {"architectures": [BOLT_ARCHITECTURE], "model_type": "t5", "d_model": d_model, "d_ff": d_ff,
            "num_heads": num_heads, "d_kv": 64, "num_layers": num_layers, "num_decoder_layers": num_decoder_layers,
            "layer_norm_epsilon": eps, "dense_act_fn": "relu", "relative_attention_num_buckets": buckets,
            "relative_attention_max_distance": max_distance, "decoder_start_token_id": 0, "reg_token_id": 1,
            "chronos_config": {"context_length": context_length, "input_patch_size": patch,
                               "input_patch_stride": patch, "prediction_length": prediction_length,
                               "quantiles": [float(v) for v in quantiles], "use_reg_token": True}}


_ENC = [("attn_norm", "encoder.block.{i}.layer.0.layer_norm.weight", "d"),
        ("q", "encoder.block.{i}.layer.0.SelfAttention.q.weight", "id"),
        ("k", "encoder.block.{i}.layer.0.SelfAttention.k.weight", "id"),
        ("v", "encoder.block.{i}.layer.0.SelfAttention.v.weight", "id"),
        ("o", "encoder.block.{i}.layer.0.SelfAttention.o.weight", "di"),
        ("ffn_norm", "encoder.block.{i}.layer.1.layer_norm.weight", "d"),
        ("wi", "encoder.block.{i}.layer.1.DenseReluDense.wi.weight", "fd"),
        ("wo", "encoder.block.{i}.layer.1.DenseReluDense.wo.weight", "df")]
_DEC = [("self_norm", "decoder.block.{i}.layer.0.layer_norm.weight", "d"),
        ("self_v", "decoder.block.{i}.layer.0.SelfAttention.v.weight", "id"),
        ("self_o", "decoder.block.{i}.layer.0.SelfAttention.o.weight", "di"),
        ("cross_norm", "decoder.block.{i}.layer.1.layer_norm.weight", "d"),
        ("cross_q", "decoder.block.{i}.layer.1.EncDecAttention.q.weight", "id"),
        ("cross_k", "decoder.block.{i}.layer.1.EncDecAttention.k.weight", "id"),
        ("cross_v", "decoder.block.{i}.layer.1.EncDecAttention.v.weight", "id"),
        ("cross_o", "decoder.block.{i}.layer.1.EncDecAttention.o.weight", "di"),
        ("ffn_norm", "decoder.block.{i}.layer.2.layer_norm.weight", "d"),
        ("wi", "decoder.block.{i}.layer.2.DenseReluDense.wi.weight", "fd"),
        ("wo", "decoder.block.{i}.layer.2.DenseReluDense.wo.weight", "df")]
_RES = [("hidden_w", "hidden_layer.weight"), ("hidden_b", "hidden_layer.bias"), ("output_w", "output_layer.weight"),
        ("output_b", "output_layer.bias"), ("residual_w", "residual_layer.weight"),
        ("residual_b", "residual_layer.bias")]


def _resblock_sizes(inp: int, hid: int, out: int) -> dict:
    return dict(hidden_w=hid * inp, hidden_b=hid, output_w=out * hid, output_b=out, residual_w=out * inp,
                residual_b=out)


def bolt_tensor_layout(c: dict) -> Dict[str, int]:
    """Every tensor the Chronos-Bolt model reads (model.zig:101-160), name -> element count."""
    d, ff, inner = c["d_model"], c["d_ff"], c["num_heads"] * c["d_kv"]
    x = c["chronos_config"]
    ps, out = x["input_patch_size"], len(x["quantiles"]) * x["prediction_length"]
    dims = {"d": d, "id": inner * d, "di": d * inner, "fd": ff * d, "df": d * ff}
    lay = {}
    for prefix, (inp, hid, o) in (("input_patch_embedding", (2 * ps, ff, d)), ("output_patch_embedding", (d, ff, out))):
        sizes = _resblock_sizes(inp, hid, o)
        for key, suffix in _RES:
            lay[f"{prefix}.{suffix}"] = sizes[key]
    lay["shared.weight"] = c["vocab"] * d
    lay["encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight"] = \
        c["relative_attention_num_buckets"] * c["num_heads"]
    lay["encoder.final_layer_norm.weight"] = d
    lay["decoder.final_layer_norm.weight"] = d
    for i in range(c["num_layers"]):
        for _, name, dim in _ENC:
            lay[name.format(i=i)] = dims[dim]
    for i in range(c["num_decoder_layers"]):
        for _, name, dim in _DEC:
            lay[name.format(i=i)] = dims[dim]
    return lay


def write_bolt_checkpoint(path: str, config: dict, weights: dict, dtype: str = "F32") -> None:
    """Write `path`/config.json and `path`/model.safetensors. `weights` in the layout the forward
    takes: reg, dec_start, rel_table (buckets, heads), enc_final_norm, dec_final_norm, enc / dec
    (lists of per-layer dicts), ie / oe (ResBlock dicts)."""
    os.makedirs(path, exist_ok=True)
    c = parse_bolt_config(json.dumps(config))
    shared = np.zeros((c["vocab"], c["d_model"]), np.float32)
    shared[c["decoder_start_token_id"]] = weights["dec_start"]
    shared[c["reg_token_id"]] = weights["reg"]
    t = {"shared.weight": shared,
         "encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight": weights["rel_table"],
         "encoder.final_layer_norm.weight": weights["enc_final_norm"],
         "decoder.final_layer_norm.weight": weights["dec_final_norm"]}
    for prefix, rb in (("input_patch_embedding", weights["ie"]), ("output_patch_embedding", weights["oe"])):
        for key, suffix in _RES:
            t[f"{prefix}.{suffix}"] = rb[key]
    for i, ly in enumerate(weights["enc"]):
        for key, name, _ in _ENC:
            t[name.format(i=i)] = ly[key]
    for i, ly in enumerate(weights["dec"]):
        for key, name, _ in _DEC:
            t[name.format(i=i)] = ly[key]
    lay = bolt_tensor_layout(c)
    for name, n in lay.items():
        if np.asarray(t[name]).size != n:
            raise ValueError(f"{name}: {np.asarray(t[name]).size} elements, the config needs {n}")
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(config, f, indent=2)
    write_safetensors(os.path.join(path, "model.safetensors"), t, dtype)


def read_bolt_weights(path: str) -> tuple:
    """(config, host weights) of a checkpoint directory, every tensor as float32 (numpy), in the
    layout write_bolt_checkpoint takes."""
    with open(os.path.join(path, "config.json")) as f:
        c = parse_bolt_config(f.read())
    d, ff, inner = c["d_model"], c["d_ff"], c["num_heads"] * c["d_kv"]
    x = c["chronos_config"]
    ps, out = x["input_patch_size"], len(x["quantiles"]) * x["prediction_length"]
    shapes = {"d": (d,), "id": (inner, d), "di": (d, inner), "fd": (ff, d), "df": (d, ff)}
    with Weights(os.path.join(path, "model.safetensors")) as w:
        def get(name, shape):
            return np.array(w.get(name, int(np.prod(shape))), np.float32).reshape(shape)

        def block(prefix, inp, hid, o):
            shp = dict(hidden_w=(hid, inp), hidden_b=(hid,), output_w=(o, hid), output_b=(o,), residual_w=(o, inp),
                       residual_b=(o,))
            return {key: get(f"{prefix}.{suffix}", shp[key]) for key, suffix in _RES}

        shared = get("shared.weight", (c["vocab"], d))
        wts = dict(reg=shared[c["reg_token_id"]].copy(), dec_start=shared[c["decoder_start_token_id"]].copy(),
                   rel_table=get("encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight",
                                 (c["relative_attention_num_buckets"], c["num_heads"])),
                   enc_final_norm=get("encoder.final_layer_norm.weight", (d,)),
                   dec_final_norm=get("decoder.final_layer_norm.weight", (d,)),
                   ie=block("input_patch_embedding", 2 * ps, ff, d), oe=block("output_patch_embedding", d, ff, out),
                   enc=[{key: get(name.format(i=i), shapes[dim]) for key, name, dim in _ENC}
                        for i in range(c["num_layers"])],
                   dec=[{key: get(name.format(i=i), shapes[dim]) for key, name, dim in _DEC}
                        for i in range(c["num_decoder_layers"])])
    return c, wts


def load_bolt(path: str, device: str = "cuda") -> "BoltForecaster":
    """A checkpoint directory (config.json + model.safetensors) as a device forecaster."""
    return BoltForecaster(path, device)


class BoltForecaster:
    """Chronos-Bolt forecaster over a local checkpoint, weights resident on the device: forecast()
    is forecaster.forecast (src/chronos_bolt/forecaster.zig:22-78) through
    tsfm_bolt_forecast_horizon."""

    def __init__(self, path: str, device: str = "cuda"):
        import torch

        self.config, host = read_bolt_weights(path)
        cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
        self.weights = dict(reg=cu(host["reg"]), dec_start=cu(host["dec_start"]), rel_table=cu(host["rel_table"]),
                            enc_final_norm=cu(host["enc_final_norm"]), dec_final_norm=cu(host["dec_final_norm"]),
                            ie={k: cu(v) for k, v in host["ie"].items()}, oe={k: cu(v) for k, v in host["oe"].items()},
                            enc=[{k: cu(v) for k, v in ly.items()} for ly in host["enc"]],
                            dec=[{k: cu(v) for k, v in ly.items()} for ly in host["dec"]])
        self.device = device

    @property
    def quantiles(self):
        return self.config["chronos_config"]["quantiles"]

    def forecast_args(self, out, inputs, horizon: int, stream=None):
        """The tsfm_bolt_horizon_args block for out (b, horizon, q) and inputs (b, t_in) device
        tensors, built once for repeated calls."""
        from . import bolt_forecast_horizon_args

        c, w = self.config, self.weights
        x = c["chronos_config"]
        return bolt_forecast_horizon_args(out, inputs, horizon, w["reg"], w["dec_start"], w["rel_table"], w["enc"],
                                          w["enc_final_norm"], w["dec"], w["dec_final_norm"], w["ie"], w["oe"],
                                          c["d_model"], c["num_heads"], c["d_ff"], c["layer_norm_epsilon"],
                                          np.asarray(x["quantiles"], np.float32), x["prediction_length"],
                                          x["context_length"], patch=x["input_patch_size"], hd=c["d_kv"],
                                          num_buckets=c["relative_attention_num_buckets"],
                                          max_distance=c["relative_attention_max_distance"], stream=stream)

    def forecast(self, inputs, horizon: int, stream=None):
        """(b, horizon, q) float32 device tensor for inputs (b, t_in) (NaN = missing)."""
        import ctypes

        import torch

        from . import OK, last_error, load

        inputs = inputs.to(self.device, torch.float32).contiguous()
        out = torch.empty((inputs.shape[0], horizon, len(self.quantiles)), dtype=torch.float32, device=self.device)
        rc = load().tsfm_bolt_forecast_horizon(ctypes.byref(self.forecast_args(out, inputs, horizon, stream)))
        if rc != OK:
            raise RuntimeError(f"tsfm_bolt_forecast_horizon: {last_error()}")
        return out
