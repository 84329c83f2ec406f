"""Python binding of libtsfm_attn.so, the gfx950 attention path of tsfm-zig.

The shared object exports the C ABI of ``include/tsfm_attn.h``; this module loads it with ctypes
and mirrors, on top of it, the reference's attention interface:

* ``Mask`` / ``Mask.pick``                 -- ``attn.Mask`` (src/core/attn.zig:10-29)
* ``Strides``                              -- ``attn.Strides`` (src/core/attn.zig:32)
* ``self_attend``                          -- ``attn.selfAttendRuntime`` for one (series, head)
                                              (src/core/attn.zig:99-117)
* ``bolt_self_attention``                  -- forRange(nb*nh, SelfJob.attend)
                                              (src/chronos_bolt/model.zig:242-243, 317-346)
* ``bolt_cross_attention``                 -- forRange(nb*nh, CrossJob.attend)
                                              (src/chronos_bolt/model.zig:296-297, 349-381)
* ``chronos2_time_attention``              -- RoPE loop + forRange(b*nh, TimeJob.attend)
                                              (src/chronos2/model.zig:236-260, 277-309)
* ``timestral_time_attention``             -- TimeJob.rope + TimeJob.attend
                                              (src/timestral/model.zig:513-515, 558-635)

Every call returns the ABI's int code: 0 = done, anything else = "not run, use the CPU path", with
``last_error()`` giving the reason -- the reference backend's contract (src/platform/backend.zig:33-36).
The ``*_checked`` helpers raise ``TsfmError`` instead. Arrays may be numpy arrays (host pointers:
the call copies in, runs and copies out synchronously) or torch device tensors (device pointers:
the call is asynchronous on the given stream). No computation happens in Python: without the
shared object or without a gfx950 device every call fails loudly.
"""
from __future__ import annotations

import ctypes
import enum
import math
import os
import pathlib
from dataclasses import dataclass
from typing import Any, Optional, Sequence

import numpy as np

LIB_PATH = pathlib.Path(__file__).with_name("libtsfm_attn.so")

OK = 0
E_UNAVAILABLE = 1
E_UNSUPPORTED = 2
E_INVALID = 3
E_DEVICE = 4

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

DEVICE_PTRS = 1
FORECAST_HOST_IO = 4  # TSFM_FORECAST_HOST_IO: the forecasts' per-call arrays in host memory
VARIATE_MAX_ROWS = 256  # TSFM_VARIATE_MAX_ROWS: rows per series of the variate and Timestral forecast calls
TIMESTRAL_BF16_ATTN = 2  # tsfm_timestral_forecast: time attention in bf16

# Every symbol include/tsfm_attn.h declares.
EXPORTS = (
    "tsfm_attn_init",
    "tsfm_attn_available",
    "tsfm_attn_fwd",
    "tsfm_attn_last_error",
    "tsfm_t5_relative_bucket",
    "tsfm_t5_bucket_table",
    "tsfm_variate_attend",
    "tsfm_qkv_project",
    "tsfm_qkv_project_noalloc",
    "tsfm_timestral_forecast",
    "tsfm_timestral_encode_categorical",
    "tsfm_chronos2_encode",
    "tsfm_chronos2_forward",
    "tsfm_bolt_forward",
    "tsfm_bolt_forecast",
    "tsfm_bolt_forecast_horizon",
    "tsfm_chronos2_forecast",
    "tsfm_weight_register",
    "tsfm_weight_release",
    "tsfm_sgemm_nt",
    "tsfm_sgemm_nn",
    "tsfm_kv_append_attend",
    "tsfm_kv_create",
    "tsfm_kv_free",
    "tsfm_kv_reset",
    "tsfm_kv_truncate",
    "tsfm_kv_len",
    "tsfm_kv_append",
    "tsfm_kv_attend",
)


class Mask(enum.IntEnum):
    """``attn.Mask`` in declaration order, plus the Timestral decoder-row mask."""

    FULL = 0
    KEYS_ADDITIVE = 1
    CAUSAL = 2
    CAUSAL_KEYS = 3
    FULL_KEYS = 4
    DECODER = 5

    @staticmethod
    def pick(causal: bool, all_keys_valid: bool, additive: bool) -> "Mask":
        """``Mask.pick`` (src/core/attn.zig:24-28)."""
        if all_keys_valid:
            return Mask.CAUSAL if causal else Mask.FULL
        if causal:
            return Mask.CAUSAL_KEYS
        return Mask.KEYS_ADDITIVE if additive else Mask.FULL_KEYS


@dataclass(frozen=True)
class Strides:
    """Token strides (elements) of q, k, v and o -- ``attn.Strides``."""

    q: int
    k: int
    v: int
    o: int


class TsfmError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"tsfm_attn error {code}: {message}")
        self.code = code


class AttnArgs(ctypes.Structure):
    """``tsfm_attn_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("mask", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("n_q", ctypes.c_int32),
        ("n_k", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("q_pos0", ctypes.c_int32),
        ("ctx_keys", ctypes.c_int32),
        ("chain_start", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("flags", ctypes.c_uint32),
        ("q", ctypes.c_void_p),
        ("q_tok", ctypes.c_int64),
        ("q_batch", ctypes.c_int64),
        ("k", ctypes.c_void_p),
        ("k_tok", ctypes.c_int64),
        ("k_batch", ctypes.c_int64),
        ("v", ctypes.c_void_p),
        ("v_tok", ctypes.c_int64),
        ("v_batch", ctypes.c_int64),
        ("o", ctypes.c_void_p),
        ("o_tok", ctypes.c_int64),
        ("o_batch", ctypes.c_int64),
        ("key_valid", ctypes.c_void_p),
        ("kv_batch", ctypes.c_int64),
        ("bias", ctypes.c_void_p),
        ("bias_head", ctypes.c_int64),
        ("bias_row", ctypes.c_int64),
        ("rel_table", ctypes.c_void_p),
        ("rel_bucket", ctypes.c_void_p),
        ("rel_buckets", ctypes.c_int32),
        ("rope_cos", ctypes.c_void_p),
        ("rope_sin", ctypes.c_void_p),
        ("rope_half", ctypes.c_int32),
        ("rope_rows_per_table", ctypes.c_int32),
        ("rope_row0", ctypes.c_int32),
        ("rope_table_stride", ctypes.c_int64),
        ("stream", ctypes.c_void_p),
    ]


_lib: Optional[ctypes.CDLL] = None


class VariateArgs(ctypes.Structure):
    """``tsfm_variate_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("groups", ctypes.c_int32),
        ("vall", ctypes.c_int32),
        ("n_tok", ctypes.c_int32),
        ("n_enc", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("cov", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("flags", ctypes.c_uint32),
        ("qkv", ctypes.c_void_p),
        ("qkv_row", ctypes.c_int64),
        ("qkv_tok", ctypes.c_int64),
        ("o", ctypes.c_void_p),
        ("o_row", ctypes.c_int64),
        ("o_tok", ctypes.c_int64),
        ("gate", ctypes.c_void_p),
        ("gate_row", ctypes.c_int64),
        ("gate_tok", ctypes.c_int64),
        ("key_valid", ctypes.c_void_p),
        ("kv_row", ctypes.c_int64),
        ("roles", ctypes.POINTER(ctypes.c_uint8)),
        ("stream", ctypes.c_void_p),
    ]


ROLE_TARGET, ROLE_PAST, ROLE_KNOWN = 0, 1, 2  # model.Role (src/timestral/model.zig:89)

CHRONOS2_LAYER_FIELDS = ("time_norm", "time_q", "time_k", "time_v", "time_o", "group_norm", "group_v", "group_o",
                         "mlp_norm", "mlp_wi", "mlp_wo")


class Chronos2Layer(ctypes.Structure):
    """``tsfm_chronos2_layer`` (include/tsfm_attn.h)."""

    _fields_ = [(f, ctypes.c_void_p) for f in CHRONOS2_LAYER_FIELDS]


RESBLOCK_FIELDS = ("hidden_w", "hidden_b", "output_w", "output_b", "residual_w", "residual_b")


class Resblock(ctypes.Structure):
    """``tsfm_resblock`` (include/tsfm_attn.h)."""

    _fields_ = [(f, ctypes.c_void_p) for f in RESBLOCK_FIELDS] + [
        ("in", ctypes.c_int32), ("hid", ctypes.c_int32), ("out", ctypes.c_int32), ("act", ctypes.c_int32)]


class TimestralAttn(ctypes.Structure):
    """``tsfm_timestral_attn`` (include/tsfm_attn.h)."""

    _fields_ = [("is_time", ctypes.c_int32), ("norm", ctypes.c_void_p), ("qkv", ctypes.c_void_p),
                ("out", ctypes.c_void_p), ("gate", ctypes.c_void_p)]


class TimestralLayer(ctypes.Structure):
    """``tsfm_timestral_layer``."""

    _fields_ = [("n_attn", ctypes.c_int32), ("attn", TimestralAttn * 2), ("mlp_norm", ctypes.c_void_p),
                ("w12", ctypes.c_void_p), ("w3", ctypes.c_void_p)]


class TimestralModel(ctypes.Structure):
    """``tsfm_timestral_model``."""

    _fields_ = [(f, ctypes.c_int32) for f in ("patch", "d_model", "heads", "head_dim", "mlp_hidden", "n_layers",
                                              "n_quantiles", "block_size", "context_length", "rope_dim",
                                              "use_asinh", "attend_missing", "covariate_enabled")] + \
               [(f, ctypes.c_float) for f in ("rope_theta", "norm_eps", "minimum_scale", "quantile_width_factor")] + \
               [("quantile_knots", ctypes.c_void_p), ("patch_proj", Resblock), ("head", Resblock),
                ("forecast_query", ctypes.c_void_p), ("out_norm", ctypes.c_void_p),
                ("layers", ctypes.POINTER(TimestralLayer))]


class TimestralForecastArgs(ctypes.Structure):
    """``tsfm_timestral_forecast_args``."""

    _fields_ = [("model", TimestralModel), ("inputs", ctypes.c_void_p), ("observed", ctypes.c_void_p)] + \
               [(f, ctypes.c_int32) for f in ("batch", "variates", "len", "horizon", "max_context", "per_shot_patches")] + \
               [("quantile_real_cap_k", ctypes.c_float), ("extreme_value_threshold", ctypes.c_float),
                ("symmetric_averaging", ctypes.c_int32), ("clip_nonnegative", ctypes.c_int32),
                ("kv_cache", ctypes.c_int32), ("flags", ctypes.c_uint32), ("out", ctypes.c_void_p),
                ("stream", ctypes.c_void_p), ("past", ctypes.c_void_p), ("known", ctypes.c_void_p),
                ("n_past", ctypes.c_int32), ("n_known", ctypes.c_int32)]


class Chronos2EncodeArgs(ctypes.Structure):
    """``tsfm_chronos2_encode_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("batch", ctypes.c_int32),
        ("seq", ctypes.c_int32),
        ("d_model", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("d_ff", ctypes.c_int32),
        ("n_layers", ctypes.c_int32),
        ("keys_all_valid", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("scale", ctypes.c_float),
        ("flags", ctypes.c_uint32),
        ("x", ctypes.c_void_p),
        ("key_valid", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p),
        ("rope_sin", ctypes.c_void_p),
        ("layers", ctypes.POINTER(Chronos2Layer)),
        ("final_norm", ctypes.c_void_p),
        ("stream", ctypes.c_void_p),
    ]


BOLT_ENC_FIELDS = ("attn_norm", "q", "k", "v", "o", "ffn_norm", "wi", "wo")
BOLT_DEC_FIELDS = ("self_norm", "self_v", "self_o", "cross_norm", "cross_q", "cross_k", "cross_v", "cross_o",
                   "ffn_norm", "wi", "wo")


class BoltEncLayer(ctypes.Structure):
    """``tsfm_bolt_enc_layer`` (include/tsfm_attn.h)."""

    _fields_ = [(f, ctypes.c_void_p) for f in BOLT_ENC_FIELDS]


class BoltDecLayer(ctypes.Structure):
    """``tsfm_bolt_dec_layer`` (include/tsfm_attn.h)."""

    _fields_ = [(f, ctypes.c_void_p) for f in BOLT_DEC_FIELDS]


class Chronos2ForwardArgs(ctypes.Structure):
    """``tsfm_chronos2_forward_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("enc", Chronos2EncodeArgs),
        ("n_ctx", ctypes.c_int32),
        ("n_out", ctypes.c_int32),
        ("feats", ctypes.c_void_p),
        ("fut_feats", ctypes.c_void_p),
        ("ctx_valid", ctypes.c_void_p),
        ("reg", ctypes.c_void_p),
        ("input_embed", Resblock),
        ("output_embed", Resblock),
        ("raw", ctypes.c_void_p),
    ]


class BoltForwardArgs(ctypes.Structure):
    """``tsfm_bolt_forward_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("batch", ctypes.c_int32),
        ("n_patch", ctypes.c_int32),
        ("d_model", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("d_ff", ctypes.c_int32),
        ("n_enc_layers", ctypes.c_int32),
        ("n_dec_layers", ctypes.c_int32),
        ("keys_all_valid", ctypes.c_int32),
        ("rel_buckets", ctypes.c_int32),
        ("rel_max_distance", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("flags", ctypes.c_uint32),
        ("feats", ctypes.c_void_p),
        ("patch_valid", ctypes.c_void_p),
        ("reg", ctypes.c_void_p),
        ("dec_start", ctypes.c_void_p),
        ("rel_table", ctypes.c_void_p),
        ("enc_layers", ctypes.POINTER(BoltEncLayer)),
        ("enc_final_norm", ctypes.c_void_p),
        ("dec_layers", ctypes.POINTER(BoltDecLayer)),
        ("dec_final_norm", ctypes.c_void_p),
        ("input_embed", Resblock),
        ("output_embed", Resblock),
        ("raw", ctypes.c_void_p),
        ("stream", ctypes.c_void_p),
    ]


class Chronos2ForecastArgs(ctypes.Structure):
    """``tsfm_chronos2_forecast_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("model", Chronos2ForwardArgs),
        ("inputs", ctypes.c_void_p),
        ("stride", ctypes.c_int64),
        ("start", ctypes.c_int64),
        ("len", ctypes.c_int32),
        ("horizon", ctypes.c_int32),
        ("time_scale", ctypes.c_float),
        ("arcsinh", ctypes.c_int32),
        ("out", ctypes.c_void_p),
    ]


class BoltHorizonArgs(ctypes.Structure):
    """``tsfm_bolt_horizon_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("model", BoltForwardArgs),
        ("inputs", ctypes.c_void_p),
        ("t_in", ctypes.c_int32),
        ("horizon", ctypes.c_int32),
        ("patch", ctypes.c_int32),
        ("prediction_length", ctypes.c_int32),
        ("context_length", ctypes.c_int32),
        ("n_quantiles", ctypes.c_int32),
        ("quantile_levels", ctypes.c_void_p),
        ("norm_eps", ctypes.c_float),
        ("out", ctypes.c_void_p),
    ]


class BoltForecastArgs(ctypes.Structure):
    """``tsfm_bolt_forecast_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("model", BoltForwardArgs),
        ("ctx", ctypes.c_void_p),
        ("stride", ctypes.c_int64),
        ("offset", ctypes.c_int64),
        ("len", ctypes.c_int32),
        ("patch", ctypes.c_int32),
        ("norm_eps", ctypes.c_float),
        ("out", ctypes.c_void_p),
    ]


class ProjArgs(ctypes.Structure):
    """``tsfm_proj_args`` (include/tsfm_attn.h)."""

    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("seq", ctypes.c_int32),
        ("d_in", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("rope_half", ctypes.c_int32),
        ("rope_rows_per_table", ctypes.c_int32),
        ("rope_row0", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("rope_table_stride", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("x_tok", ctypes.c_int64),
        ("w_q", ctypes.c_void_p),
        ("w_k", ctypes.c_void_p),
        ("w_v", ctypes.c_void_p),
        ("w_gate", ctypes.c_void_p),
        ("q", ctypes.c_void_p),
        ("q_tok", ctypes.c_int64),
        ("k", ctypes.c_void_p),
        ("k_tok", ctypes.c_int64),
        ("v", ctypes.c_void_p),
        ("v_tok", ctypes.c_int64),
        ("gate", ctypes.c_void_p),
        ("gate_tok", ctypes.c_int64),
        ("rope_cos", ctypes.c_void_p),
        ("rope_sin", ctypes.c_void_p),
        ("stream", ctypes.c_void_p),
    ]


def load(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Load libtsfm_attn.so (built in-tree by ``make -C tsfm-zig_amd``). Raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built: run `make -C tsfm-zig_amd` (or __graft_entry__.build())")
    # A process must hold exactly one HIP runtime. torch wheels bundle their own libamdhip64
    # (soname libamdhip64.so.7) and their HIP libraries ask for it by the unversioned name, so a
    # system runtime loaded first (by this library) would not satisfy them and torch would load a
    # second one, under which it sees no device and its streams mean nothing to this library.
    # Loading torch first lets this library's libamdhip64.so.7 dependency bind to torch's copy.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(p))
    vp, i32, i64, u32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
    lib.tsfm_attn_init.restype = ctypes.c_int
    lib.tsfm_attn_available.restype = ctypes.c_int
    lib.tsfm_attn_fwd.argtypes = [ctypes.POINTER(AttnArgs)]
    lib.tsfm_attn_fwd.restype = ctypes.c_int
    lib.tsfm_attn_last_error.restype = ctypes.c_char_p
    lib.tsfm_t5_relative_bucket.argtypes = [i64, u32, u32]
    lib.tsfm_t5_relative_bucket.restype = u32
    lib.tsfm_t5_bucket_table.argtypes = [vp, i32, i32, u32, u32]
    lib.tsfm_t5_bucket_table.restype = ctypes.c_int
    lib.tsfm_kv_create.argtypes = [ctypes.POINTER(vp), i32, i32, i32, i32, i32]
    lib.tsfm_kv_create.restype = ctypes.c_int
    lib.tsfm_kv_free.argtypes = [vp]
    lib.tsfm_kv_free.restype = ctypes.c_int
    lib.tsfm_kv_reset.argtypes = [vp]
    lib.tsfm_kv_reset.restype = ctypes.c_int
    lib.tsfm_kv_append_attend.argtypes = [vp, vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, i32,
                                          ctypes.c_float, u32, vp]
    lib.tsfm_kv_append_attend.restype = ctypes.c_int
    lib.tsfm_kv_truncate.argtypes = [vp, i32]
    lib.tsfm_kv_truncate.restype = ctypes.c_int
    lib.tsfm_kv_len.argtypes = [vp]
    lib.tsfm_kv_len.restype = i32
    lib.tsfm_kv_append.argtypes = [vp, vp, i64, i64, vp, i64, i64, i32, u32, vp]
    lib.tsfm_kv_append.restype = ctypes.c_int
    lib.tsfm_kv_attend.argtypes = [vp, vp, i64, i64, vp, i64, i64, i32, i32, ctypes.c_float, u32, vp]
    lib.tsfm_kv_attend.restype = ctypes.c_int
    lib.tsfm_variate_attend.argtypes = [ctypes.POINTER(VariateArgs)]
    lib.tsfm_variate_attend.restype = ctypes.c_int
    lib.tsfm_qkv_project.argtypes = [ctypes.POINTER(ProjArgs)]
    lib.tsfm_qkv_project.restype = ctypes.c_int
    lib.tsfm_qkv_project_noalloc.argtypes = [ctypes.POINTER(ProjArgs)]
    lib.tsfm_qkv_project_noalloc.restype = ctypes.c_int
    lib.tsfm_chronos2_encode.argtypes = [ctypes.POINTER(Chronos2EncodeArgs)]
    lib.tsfm_chronos2_encode.restype = ctypes.c_int
    lib.tsfm_chronos2_forward.argtypes = [ctypes.POINTER(Chronos2ForwardArgs)]
    lib.tsfm_chronos2_forward.restype = ctypes.c_int
    lib.tsfm_bolt_forward.argtypes = [ctypes.POINTER(BoltForwardArgs)]
    lib.tsfm_bolt_forward.restype = ctypes.c_int
    lib.tsfm_bolt_forecast.argtypes = [ctypes.POINTER(BoltForecastArgs)]
    lib.tsfm_bolt_forecast.restype = ctypes.c_int
    lib.tsfm_bolt_forecast_horizon.argtypes = [ctypes.POINTER(BoltHorizonArgs)]
    lib.tsfm_bolt_forecast_horizon.restype = ctypes.c_int
    lib.tsfm_chronos2_forecast.argtypes = [ctypes.POINTER(Chronos2ForecastArgs)]
    lib.tsfm_chronos2_forecast.restype = ctypes.c_int
    lib.tsfm_timestral_forecast.argtypes = [ctypes.POINTER(TimestralForecastArgs)]
    lib.tsfm_timestral_forecast.restype = ctypes.c_int
    lib.tsfm_timestral_encode_categorical.argtypes = [ctypes.POINTER(CategoricalArgs)]
    lib.tsfm_timestral_encode_categorical.restype = ctypes.c_int
    lib.tsfm_weight_register.argtypes = [vp, ctypes.c_size_t]
    lib.tsfm_weight_register.restype = vp
    lib.tsfm_weight_release.argtypes = [vp]
    lib.tsfm_weight_release.restype = None
    ci, cf = ctypes.c_int, ctypes.c_float
    lib.tsfm_sgemm_nt.argtypes = [ci, ci, ci, cf, vp, ci, vp, ci, vp, ci, vp]
    lib.tsfm_sgemm_nt.restype = ci
    lib.tsfm_sgemm_nn.argtypes = [ci, ci, ci, vp, ci, vp, ci, vp, ci, vp]
    lib.tsfm_sgemm_nn.restype = ci
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    return load().tsfm_attn_last_error().decode()


def available() -> bool:
    return bool(load().tsfm_attn_available())


def _ptr(x: Any) -> Optional[int]:
    """Address of a numpy array, a torch tensor, or an int; None stays None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        if not x.flags["C_CONTIGUOUS"]:
            raise ValueError("numpy arrays passed to tsfm_attn must be C-contiguous")
        return x.ctypes.data
    raise TypeError(f"cannot take the address of {type(x)}")


def _is_device(x: Any) -> bool:
    return hasattr(x, "is_cuda") and bool(x.is_cuda)


def _dtype_code(x: Any) -> int:
    name = str(getattr(x, "dtype", "float32"))
    if "bfloat16" in name:
        return DTYPE_BF16
    if "float16" in name:
        return DTYPE_F16
    if "float32" in name:
        return DTYPE_F32
    raise TypeError(f"unsupported element type {name}")


def _stream_of(x: Any, stream: Any) -> Optional[int]:
    if stream is not None:
        return int(getattr(stream, "cuda_stream", stream))
    if _is_device(x):
        import torch  # device-pointer calls run on torch's current stream by default

        return int(torch.cuda.current_stream(x.device).cuda_stream)
    return None


def fwd(args: AttnArgs) -> int:
    """``tsfm_attn_fwd``: returns the ABI code."""
    return int(load().tsfm_attn_fwd(ctypes.byref(args)))


def fwd_checked(args: AttnArgs) -> None:
    rc = fwd(args)
    if rc != OK:
        raise TsfmError(rc, last_error())


def make_args(
    *,
    q: Any,
    k: Any,
    v: Any,
    o: Any,
    mask: int,
    batch: int,
    heads: int,
    n_q: int,
    n_k: int,
    q_tok: int,
    q_batch: int,
    k_tok: int,
    k_batch: int,
    v_tok: int,
    v_batch: int,
    o_tok: int,
    o_batch: int,
    scale: float,
    head_dim: int = 64,
    q_pos0: int = 0,
    ctx_keys: int = 0,
    chain_start: int = 0,
    key_valid: Any = None,
    kv_batch: int = 0,
    bias: Any = None,
    bias_head: int = 0,
    bias_row: int = 0,
    rel_table: Any = None,
    rel_bucket: Any = None,
    rel_buckets: int = 0,
    rope_cos: Any = None,
    rope_sin: Any = None,
    rope_rows_per_table: int = 0,
    rope_row0: int = 0,
    rope_table_stride: int = 0,
    stream: Any = None,
    dtype: Optional[int] = None,
) -> AttnArgs:
    """Build ``tsfm_attn_args``; device mode is chosen when q is a device tensor."""
    device = _is_device(q)
    a = AttnArgs()
    a.dtype = _dtype_code(q) if dtype is None else dtype
    a.mask = int(mask)
    a.batch, a.heads, a.n_q, a.n_k, a.head_dim = batch, heads, n_q, n_k, head_dim
    a.q_pos0, a.ctx_keys, a.chain_start = q_pos0, ctx_keys, chain_start
    a.scale = float(scale)
    a.flags = DEVICE_PTRS if device else 0
    a.q, a.q_tok, a.q_batch = _ptr(q), q_tok, q_batch
    a.k, a.k_tok, a.k_batch = _ptr(k), k_tok, k_batch
    a.v, a.v_tok, a.v_batch = _ptr(v), v_tok, v_batch
    a.o, a.o_tok, a.o_batch = _ptr(o), o_tok, o_batch
    a.key_valid, a.kv_batch = _ptr(key_valid), kv_batch
    a.bias, a.bias_head, a.bias_row = _ptr(bias), bias_head, bias_row
    a.rel_table, a.rel_bucket, a.rel_buckets = _ptr(rel_table), _ptr(rel_bucket), rel_buckets
    a.rope_cos, a.rope_sin = _ptr(rope_cos), _ptr(rope_sin)
    a.rope_half = head_dim // 2 if rope_cos is not None else 0
    a.rope_rows_per_table, a.rope_row0, a.rope_table_stride = rope_rows_per_table, rope_row0, rope_table_stride
    a.stream = _stream_of(q, stream) if device else None
    return a


def _flat_view(x: Any, offset: int) -> Any:
    """x shifted by `offset` elements (numpy view or torch view)."""
    if offset == 0:
        return x
    return x.reshape(-1)[offset:]


# ---------------------------------------------------------------------------------------------
# Mirrors of the reference call sites.


def self_attend(mask: Mask, q, k, v, o, st: Strides, n: int, hd: int, scale: float, key_valid=None, bias=None) -> int:
    """``attn.selfAttendRuntime`` for one (series, head): q/k/v/o start at the head's first element,
    ``st`` gives token strides, ``bias`` is an optional (n, n) additive bias."""
    return fwd(
        make_args(
            q=q, k=k, v=v, o=o, mask=mask, batch=1, heads=1, n_q=n, n_k=n, head_dim=hd,
            q_tok=st.q, q_batch=0, k_tok=st.k, k_batch=0, v_tok=st.v, v_batch=0, o_tok=st.o, o_batch=0,
            scale=scale, key_valid=key_valid, kv_batch=0, bias=bias, bias_head=0, bias_row=n,
        )
    )


def bolt_self_attention(q, k, v, o, rel_table, rel_bucket, key_valid, keys_all_valid: bool, nb: int, seq: int,
                        inner: int, nh: int, hd: int, num_buckets: int, stream=None) -> int:
    """Chronos-Bolt encoder self-attention over all (series, head): no scale, T5 bias from the
    (buckets, heads) table, additive key mask unless every key of the chunk is valid."""
    mask = Mask.pick(False, keys_all_valid, True)
    return fwd(
        make_args(
            q=q, k=k, v=v, o=o, mask=mask, batch=nb, heads=nh, n_q=seq, n_k=seq, head_dim=hd,
            q_tok=inner, q_batch=seq * inner, k_tok=inner, k_batch=seq * inner, v_tok=inner, v_batch=seq * inner,
            o_tok=inner, o_batch=seq * inner, scale=1.0, key_valid=key_valid, kv_batch=seq,
            rel_table=rel_table, rel_bucket=rel_bucket, rel_buckets=num_buckets, stream=stream,
        )
    )


def bolt_cross_attention(q, k, v, o, key_valid, nb: int, seq: int, inner: int, nh: int, hd: int, stream=None) -> int:
    """Chronos-Bolt decoder cross-attention: one query per (series, head), additive key mask."""
    return fwd(
        make_args(
            q=q, k=k, v=v, o=o, mask=Mask.KEYS_ADDITIVE, batch=nb, heads=nh, n_q=1, n_k=seq, head_dim=hd,
            q_tok=inner, q_batch=inner, k_tok=inner, k_batch=seq * inner, v_tok=inner, v_batch=seq * inner,
            o_tok=inner, o_batch=inner, scale=1.0, key_valid=key_valid, kv_batch=seq, stream=stream,
        )
    )


def chronos2_time_attention(q, k, v, o, cos_t, sin_t, key_valid, keys_all_valid: bool, b: int, seq: int, d: int,
                            nh: int, hd: int, scale: float = 1.0, stream=None) -> int:
    """Chronos-2 time attention: RoPE on q and k (tables (seq, hd/2)), then non-causal attention with
    the additive key mask. The model uses scale 1.0 (src/chronos2/model.zig:306)."""
    mask = Mask.pick(False, keys_all_valid, True)
    return fwd(
        make_args(
            q=q, k=k, v=v, o=o, mask=mask, batch=b, heads=nh, n_q=seq, n_k=seq, head_dim=hd,
            q_tok=d, q_batch=seq * d, k_tok=d, k_batch=seq * d, v_tok=d, v_batch=seq * d, o_tok=d, o_batch=seq * d,
            scale=scale, key_valid=key_valid, kv_batch=seq, rope_cos=cos_t, rope_sin=sin_t, stream=stream,
        )
    )


def timestral_time_attention(qkv, o, cos_t, sin_t, key_valid, keys_all_valid: bool, bidir: Optional[Sequence[bool]],
                             rows: int, vall: int, ne: int, l: int, h: int, d: int, nh: int, hd: int,
                             stream=None) -> int:
    """Timestral time attention over [Enc ; Dec] tokens of every row: RoPE (per-group tables
    (groups, sl, hd/2)), encoder rows causal (or bidirectional for known-future rows), decoder rows
    over valid context keys plus their own causal chain. qkv is (rows, sl, 3d), o is (rows, sl, d)."""
    sl = ne + h
    scale = 1.0 / math.sqrt(hd)
    flags = [bool(x) for x in bidir] if bidir is not None else [False] * rows
    common = dict(heads=nh, head_dim=hd, scale=scale, rope_cos=cos_t, rope_sin=sin_t, rope_rows_per_table=vall,
                  rope_table_stride=sl * (hd // 2), stream=stream, q_tok=3 * d, k_tok=3 * d, v_tok=3 * d, o_tok=d,
                  q_batch=sl * 3 * d, k_batch=sl * 3 * d, v_batch=sl * 3 * d, o_batch=sl * d,
                  key_valid=key_valid, kv_batch=ne)
    # Encoder rows, grouped into runs of rows with the same causality (rows of one run share a call).
    r = 0
    while r < rows:
        r1 = r
        while r1 < rows and flags[r1] == flags[r]:
            r1 += 1
        mask = Mask.pick(not flags[r], keys_all_valid, False)
        rc = fwd(make_args(
            q=_flat_view(qkv, r * sl * 3 * d), k=_flat_view(qkv, r * sl * 3 * d + d),
            v=_flat_view(qkv, r * sl * 3 * d + 2 * d), o=_flat_view(o, r * sl * d), mask=mask, batch=r1 - r,
            n_q=ne, n_k=ne, rope_row0=r, **{**common, "key_valid": _flat_view(key_valid, r * ne)}))
        if rc != OK:
            return rc
        r = r1
    if h == 0:
        return OK
    # Decoder rows: queries at [ne, sl), keys [0, sl).
    return fwd(make_args(
        q=_flat_view(qkv, ne * 3 * d), k=_flat_view(qkv, d), v=_flat_view(qkv, 2 * d), o=_flat_view(o, ne * d),
        mask=Mask.DECODER, batch=rows, n_q=h, n_k=sl, q_pos0=ne, ctx_keys=l, chain_start=ne,
        **{**common, "key_valid": key_valid}))


def variate_attend(args: VariateArgs) -> int:
    """``tsfm_variate_attend``: returns the ABI code."""
    return int(load().tsfm_variate_attend(ctypes.byref(args)))


def timestral_variate_attention(qkv, o, key_valid, roles: Sequence[int], cov: bool, groups: int, vall: int, ne: int,
                                h: int, d: int, nh: int, hd: int, gate=None, stream=None) -> int:
    """Timestral variate attention (Model.variateAttention, src/timestral/model.zig:525-544): the
    forRangeMin(groups * sl, VariateJob.run) call and, with ``gate``, the nn.mulSigmoid after it.
    qkv is (groups * vall, sl, 3d) in the permuted (token, qkv, head, hd) layout, o and gate are
    (groups * vall, sl, d), key_valid (groups * vall, ne); ``roles`` holds vall model.Role values.
    Device tensors run asynchronously on ``stream`` (default: torch's current stream); numpy arrays
    are staged through the library and the call returns when o is written."""
    sl = ne + h
    device = _is_device(qkv)
    role_list = [int(r) for r in roles]
    role_bytes = (ctypes.c_uint8 * max(len(role_list), 1))(*role_list)
    a = VariateArgs(dtype=_dtype_code(qkv), groups=groups, vall=vall, n_tok=sl, n_enc=ne, heads=nh, head_dim=hd,
                    cov=int(bool(cov)), scale=1.0 / math.sqrt(hd), flags=DEVICE_PTRS if device else 0,
                    qkv=_ptr(qkv), qkv_row=sl * 3 * d, qkv_tok=3 * d, o=_ptr(o), o_row=sl * d, o_tok=d,
                    gate=_ptr(gate), gate_row=sl * d if gate is not None else 0, gate_tok=d if gate is not None else 0,
                    key_valid=_ptr(key_valid), kv_row=ne, roles=role_bytes,
                    stream=_stream_of(qkv, stream) if device else None)
    return variate_attend(a)


def qkv_project(args: ProjArgs) -> int:
    """``tsfm_qkv_project``: returns the ABI code."""
    return int(load().tsfm_qkv_project(ctypes.byref(args)))


def qkv_project_noalloc(args: ProjArgs) -> int:
    """``tsfm_qkv_project_noalloc`` (device pointers; allocates nothing): returns the ABI code."""
    return int(load().tsfm_qkv_project_noalloc(ctypes.byref(args)))


def _proj(x, wq, wk, wv, q, k, v, *, batch: int, seq: int, d_in: int, nh: int, hd: int, x_tok: int, y_tok: int,
          cos_t=None, sin_t=None, rope_rows_per_table: int = 0, rope_row0: int = 0, rope_table_stride: int = 0,
          w_gate=None, gate=None, gate_tok: int = 0, stream=None) -> int:
    device = _is_device(x)
    a = ProjArgs(dtype=_dtype_code(x), out_dtype=_dtype_code(q), batch=batch, seq=seq, d_in=d_in, heads=nh, head_dim=hd,
                 flags=DEVICE_PTRS if device else 0, rope_half=hd // 2 if cos_t is not None else 0,
                 rope_rows_per_table=rope_rows_per_table, rope_row0=rope_row0, rope_table_stride=rope_table_stride,
                 x=_ptr(x), x_tok=x_tok, w_q=_ptr(wq), w_k=_ptr(wk), w_v=_ptr(wv), w_gate=_ptr(w_gate),
                 q=_ptr(q), q_tok=y_tok, k=_ptr(k), k_tok=y_tok, v=_ptr(v), v_tok=y_tok, gate=_ptr(gate),
                 gate_tok=gate_tok, rope_cos=_ptr(cos_t), rope_sin=_ptr(sin_t),
                 stream=_stream_of(x, stream) if device else None)
    return qkv_project(a)


def chronos2_qkv_projection(xn, wq, wk, wv, q, k, v, cos_t, sin_t, b: int, seq: int, d: int, nh: int, hd: int,
                            stream=None) -> int:
    """Chronos-2 time-attention projections (src/chronos2/model.zig:232-245): q, k, v =
    nn.linear(xn, W) for the three (d, d) weights, then RoPE on every head of q and k with the
    (seq, hd/2) tables. xn, q, k, v are (b * seq, d)."""
    return _proj(xn, wq, wk, wv, q, k, v, batch=b, seq=seq, d_in=d, nh=nh, hd=hd, x_tok=d, y_tok=d, cos_t=cos_t,
                 sin_t=sin_t, stream=stream)


def timestral_qkv_projection(xn, w_qkv, qkv, cos_t, sin_t, rows: int, vall: int, sl: int, d: int, nh: int, hd: int,
                             w_gate=None, gate=None, stream=None) -> int:
    """Timestral time-attention projections (src/timestral/model.zig:494-500,513): the fused qkv
    nn.linear over the permuted (3d, d) weight into qkv (rows * sl, 3d), TimeJob.rope on its q and k
    heads with the per-group (groups, sl, hd/2) tables, and with ``w_gate`` the gate nn.linear into
    gate (rows * sl, d)."""
    return _proj(xn, w_qkv, _flat_view(w_qkv, d * d), _flat_view(w_qkv, 2 * d * d), qkv, _flat_view(qkv, d),
                 _flat_view(qkv, 2 * d), batch=rows, seq=sl, d_in=d, nh=nh, hd=hd, x_tok=d, y_tok=3 * d,
                 cos_t=cos_t, sin_t=sin_t, rope_rows_per_table=vall, rope_table_stride=sl * (hd // 2),
                 w_gate=w_gate, gate=gate, gate_tok=d if gate is not None else 0, stream=stream)


def bolt_qkv_projection(x, wq, wk, wv, q, k, v, nb: int, seq: int, d: int, nh: int, hd: int, stream=None) -> int:
    """Chronos-Bolt encoder self-attention projections (src/chronos_bolt/model.zig:239-241): q, k,
    v = nn.linear(x, W) with (inner, d) weights, inner = nh * hd; no RoPE."""
    return _proj(x, wq, wk, wv, q, k, v, batch=nb, seq=seq, d_in=d, nh=nh, hd=hd, x_tok=d, y_tok=nh * hd,
                 stream=stream)


def chronos2_encode(x, key_valid, cos_t, sin_t, layers: Sequence[dict], final_norm, b: int, seq: int, d: int,
                    nh: int, d_ff: int, eps: float, keys_all_valid: Optional[bool] = None, scale: float = 1.0,
                    hd: int = 64, stream=None) -> int:
    """Chronos-2 ``Model.encode`` layer loop and final norm (src/chronos2/model.zig:144-206) in one
    call: x (b * seq, d) embedded tokens in, hidden states out (in place); layers: one dict per
    layer of the CHRONOS2_LAYER_FIELDS arrays. ``keys_all_valid`` defaults to the AND of key_valid
    (computed here for host arrays; device callers pass it, as the reference's caller does)."""
    device = _is_device(x)
    if keys_all_valid is None:
        if device:
            raise ValueError("keys_all_valid is required with device tensors")
        keys_all_valid = bool(np.asarray(key_valid).all())
    arr = (Chronos2Layer * max(1, len(layers)))()
    for i, ly in enumerate(layers):
        for f in CHRONOS2_LAYER_FIELDS:
            setattr(arr[i], f, _ptr(ly[f]))
    a = Chronos2EncodeArgs(batch=b, seq=seq, d_model=d, heads=nh, head_dim=hd, d_ff=d_ff, n_layers=len(layers),
                           keys_all_valid=int(bool(keys_all_valid)), eps=eps, scale=scale,
                           flags=DEVICE_PTRS if device else 0, x=_ptr(x), key_valid=_ptr(key_valid),
                           rope_cos=_ptr(cos_t), rope_sin=_ptr(sin_t), layers=arr, final_norm=_ptr(final_norm),
                           stream=_stream_of(x, stream) if device else None)
    return int(load().tsfm_chronos2_encode(ctypes.byref(a)))


def _resblock(rb: dict, act: int = 0) -> Resblock:
    st = Resblock(act=act)
    for f in RESBLOCK_FIELDS:
        setattr(st, f, _ptr(rb.get(f)))
    hid, d_in = (int(x) for x in rb["hidden_w"].shape)
    st.hid = hid
    setattr(st, "in", d_in)
    st.out = int(rb["output_w"].shape[0])
    return st


def chronos2_forward(raw, feats, fut_feats, ctx_valid, reg, cos_t, sin_t, layers: Sequence[dict], final_norm,
                     input_embed: dict, output_embed: dict, b: int, n_ctx: int, n_out: int, d: int, nh: int,
                     d_ff: int, eps: float, keys_all_valid: Optional[bool] = None, scale: float = 1.0, hd: int = 64,
                     stream=None) -> int:
    """The model part of the Chronos-2 forecaster (src/chronos2/forecaster.zig:155-183) in one
    call: input embedding of the context and future patch features, [context; REG; future], the
    encoder stack, the future rows, the output head into raw (b * n_out, head out). The ResBlocks are
    dicts of RESBLOCK_FIELDS arrays; ``keys_all_valid`` (of the context patches) defaults to the
    AND of ctx_valid for host arrays."""
    device = _is_device(feats)
    if keys_all_valid is None:
        if device:
            raise ValueError("keys_all_valid is required with device tensors")
        keys_all_valid = bool(np.asarray(ctx_valid).all())
    a = _chronos2_args(raw, feats, fut_feats, ctx_valid, reg, cos_t, sin_t, layers, final_norm, input_embed,
                       output_embed, b, n_ctx, n_out, d, nh, d_ff, eps, keys_all_valid, scale, hd, device, stream)
    return int(load().tsfm_chronos2_forward(ctypes.byref(a)))


def _chronos2_args(raw, feats, fut_feats, ctx_valid, reg, cos_t, sin_t, layers, final_norm, input_embed, output_embed,
                   b, n_ctx, n_out, d, nh, d_ff, eps, keys_all_valid, scale, hd, device, stream):
    arr = (Chronos2Layer * max(1, len(layers)))()
    for i, ly in enumerate(layers):
        for f in CHRONOS2_LAYER_FIELDS:
            setattr(arr[i], f, _ptr(ly[f]))
    enc = Chronos2EncodeArgs(batch=b, seq=n_ctx + 1 + n_out, d_model=d, heads=nh, head_dim=hd, d_ff=d_ff,
                             n_layers=len(layers), keys_all_valid=int(bool(keys_all_valid)), eps=eps, scale=scale,
                             flags=DEVICE_PTRS if device else 0, rope_cos=_ptr(cos_t), rope_sin=_ptr(sin_t),
                             layers=arr, final_norm=_ptr(final_norm),
                             stream=_stream_of(reg, stream) if device else None)
    a = Chronos2ForwardArgs(enc=enc, n_ctx=n_ctx, n_out=n_out, feats=_ptr(feats), fut_feats=_ptr(fut_feats),
                            ctx_valid=_ptr(ctx_valid), reg=_ptr(reg), input_embed=_resblock(input_embed),
                            output_embed=_resblock(output_embed), raw=_ptr(raw))
    a._keep = arr  # the layer array must outlive the call
    return a


def chronos2_forecast(out, inputs, length: int, horizon: int, reg, cos_t, sin_t, layers: Sequence[dict], final_norm,
                      input_embed: dict, output_embed: dict, n: int, d: int, nh: int, d_ff: int, eps: float,
                      patch: int = 16, stride: Optional[int] = None, start: int = 0, time_scale: float = 1.0,
                      arcsinh: bool = False, scale: float = 1.0, hd: int = 64, stream=None) -> int:
    """The whole Chronos-2 forecast of n series on device tensors (runChunk,
    src/chronos2/forecaster.zig:59-204): row s is inputs[s * stride + start:][:length] (NaN =
    missing); out (n, horizon, q) receives the quantile forecasts in data units. cos_t / sin_t are
    the (n_ctx + 1 + n_out, 32) RoPE tables of the sequence."""
    a = chronos2_forecast_args(out, inputs, length, horizon, reg, cos_t, sin_t, layers, final_norm, input_embed,
                               output_embed, n, d, nh, d_ff, eps, patch, stride, start, time_scale, arcsinh, scale, hd,
                               stream)
    return int(load().tsfm_chronos2_forecast(ctypes.byref(a)))


def chronos2_forecast_args(out, inputs, length, horizon, reg, cos_t, sin_t, layers, final_norm, input_embed,
                           output_embed, n, d, nh, d_ff, eps, patch=16, stride=None, start=0, time_scale=1.0,
                           arcsinh=False, scale=1.0, hd=64, stream=None) -> Chronos2ForecastArgs:
    """The argument block of chronos2_forecast, built once for repeated tsfm_chronos2_forecast calls
    (the layer array it points to lives as long as the returned object)."""
    n_ctx, n_out = (length + patch - 1) // patch, (horizon + patch - 1) // patch
    m = _chronos2_args(None, None, None, None, reg, cos_t, sin_t, layers, final_norm, input_embed, output_embed, n,
                       n_ctx, n_out, d, nh, d_ff, eps, False, scale, hd, True, stream)
    if not _is_device(inputs):  # host inputs and out, device weights: TSFM_FORECAST_HOST_IO
        m.enc.flags |= FORECAST_HOST_IO
    a = Chronos2ForecastArgs(model=m, inputs=_ptr(inputs), stride=length if stride is None else stride, start=start,
                             len=length, horizon=horizon, time_scale=time_scale, arcsinh=int(bool(arcsinh)),
                             out=_ptr(out))
    a._keep = (m._keep, inputs, out)
    return a


def bolt_forward(raw, feats, patch_valid, reg, dec_start, rel_table, enc_layers: Sequence[dict], enc_final_norm,
                 dec_layers: Sequence[dict], dec_final_norm, input_embed: dict, output_embed: dict, b: int,
                 n_patch: int, d: int, nh: int, d_ff: int, eps: float, num_buckets: int = 32, max_distance: int = 128,
                 keys_all_valid: Optional[bool] = None, hd: int = 64, stream=None) -> int:
    """The model part of the Chronos-Bolt forecaster (src/chronos_bolt/forecaster.zig:199-213) in one
    call: input embedding of the [values, mask] patch features, [patches; REG], the T5 encoder with
    the relative position bias, the one-token decoder with cross-attention, the output head into
    raw (b, head out). Layers are dicts of BOLT_ENC_FIELDS / BOLT_DEC_FIELDS arrays."""
    device = _is_device(feats)
    if keys_all_valid is None:
        if device:
            raise ValueError("keys_all_valid is required with device tensors")
        keys_all_valid = bool(np.asarray(patch_valid).all())
    a = bolt_forward_args(enc_layers, dec_layers, feats, patch_valid, reg, dec_start, rel_table, enc_final_norm, dec_final_norm, input_embed,
                   output_embed, raw, b, n_patch, d, nh, hd, d_ff, eps, num_buckets, max_distance, keys_all_valid,
                   device, stream)
    return int(load().tsfm_bolt_forward(ctypes.byref(a)))


def bolt_forward_args(enc_layers, dec_layers, feats, patch_valid, reg, dec_start, rel_table, enc_final_norm,
                      dec_final_norm, input_embed, output_embed, raw, b, n_patch, d, nh, hd, d_ff, eps, num_buckets,
                      max_distance, keys_all_valid, device, stream) -> BoltForwardArgs:
    """The argument block of bolt_forward, built once for repeated tsfm_bolt_forward calls (the
    layer arrays it points to live as long as the returned object)."""
    ea = (BoltEncLayer * max(1, len(enc_layers)))()
    for i, ly in enumerate(enc_layers):
        for f in BOLT_ENC_FIELDS:
            setattr(ea[i], f, _ptr(ly[f]))
    da = (BoltDecLayer * max(1, len(dec_layers)))()
    for i, ly in enumerate(dec_layers):
        for f in BOLT_DEC_FIELDS:
            setattr(da[i], f, _ptr(ly[f]))
    a = BoltForwardArgs(batch=b, n_patch=n_patch, d_model=d, heads=nh, head_dim=hd, d_ff=d_ff,
                        n_enc_layers=len(enc_layers), n_dec_layers=len(dec_layers),
                        keys_all_valid=int(bool(keys_all_valid)), rel_buckets=num_buckets,
                        rel_max_distance=max_distance, eps=eps, flags=DEVICE_PTRS if device else 0, feats=_ptr(feats),
                        patch_valid=_ptr(patch_valid), reg=_ptr(reg), dec_start=_ptr(dec_start),
                        rel_table=_ptr(rel_table), enc_layers=ea, enc_final_norm=_ptr(enc_final_norm), dec_layers=da,
                        dec_final_norm=_ptr(dec_final_norm), input_embed=_resblock(input_embed),
                        output_embed=_resblock(output_embed), raw=_ptr(raw),
                        stream=_stream_of(reg, stream) if device else None)
    a._keep = (ea, da)
    return a


def bolt_forecast(out, ctx, length: int, reg, dec_start, rel_table, enc_layers: Sequence[dict], enc_final_norm,
                  dec_layers: Sequence[dict], dec_final_norm, input_embed: dict, output_embed: dict, n: int, d: int,
                  nh: int, d_ff: int, eps: float, patch: int = 16, stride: Optional[int] = None, offset: int = 0,
                  norm_eps: float = 1e-5, num_buckets: int = 32, max_distance: int = 128, hd: int = 64,
                  stream=None) -> int:
    """The whole Chronos-Bolt forecast of n series on device tensors (predictBlock/runChunk,
    src/chronos_bolt/forecaster.zig:115-220): row s of the context is ctx[s * stride + offset:][:length]
    (NaN = missing); out (n, q * P) receives the quantile forecasts in data units."""
    a = bolt_forecast_args(out, ctx, length, reg, dec_start, rel_table, enc_layers, enc_final_norm, dec_layers,
                           dec_final_norm, input_embed, output_embed, n, d, nh, d_ff, eps, patch, stride, offset,
                           norm_eps, num_buckets, max_distance, hd, stream)
    return int(load().tsfm_bolt_forecast(ctypes.byref(a)))


def bolt_forecast_args(out, ctx, length, reg, dec_start, rel_table, enc_layers, enc_final_norm, dec_layers,
                       dec_final_norm, input_embed, output_embed, n, d, nh, d_ff, eps, patch=16, stride=None, offset=0,
                       norm_eps=1e-5, num_buckets=32, max_distance=128, hd=64, stream=None) -> BoltForecastArgs:
    """The argument block of bolt_forecast, built once: a caller that forecasts repeatedly with the
    same weights and buffers passes it to tsfm_bolt_forecast each time (the layer arrays it points
    to live as long as the returned object)."""
    n_patch = (length + patch - 1) // patch
    m = bolt_forward_args(enc_layers, dec_layers, None, None, reg, dec_start, rel_table, enc_final_norm, dec_final_norm,
                   input_embed, output_embed, None, n, n_patch, d, nh, hd, d_ff, eps, num_buckets, max_distance, False,
                   True, stream)
    if not _is_device(ctx):  # host context and out, device weights: TSFM_FORECAST_HOST_IO
        m.flags |= FORECAST_HOST_IO
    a = BoltForecastArgs(model=m, ctx=_ptr(ctx), stride=length if stride is None else stride, offset=offset,
                         len=length, patch=patch, norm_eps=norm_eps, out=_ptr(out))
    a._keep = (m._keep, ctx, out)
    return a


def bolt_forecast_horizon(out, inputs, horizon: int, reg, dec_start, rel_table, enc_layers: Sequence[dict],
                          enc_final_norm, dec_layers: Sequence[dict], dec_final_norm, input_embed: dict,
                          output_embed: dict, d: int, nh: int, d_ff: int, eps: float, quantile_levels,
                          prediction_length: int, context_length: int, patch: int = 16, norm_eps: float = 1e-5,
                          num_buckets: int = 32, max_distance: int = 128, hd: int = 64, stream=None) -> int:
    """Chronos-Bolt forecaster.forecast (src/chronos_bolt/forecaster.zig:22-78) on device tensors,
    any horizon: inputs (b, t_in) f32 (NaN = missing), out (b, horizon, q). Returns the ABI code."""
    a = bolt_forecast_horizon_args(out, inputs, horizon, reg, dec_start, rel_table, enc_layers, enc_final_norm,
                                   dec_layers, dec_final_norm, input_embed, output_embed, d, nh, d_ff, eps,
                                   quantile_levels, prediction_length, context_length, patch, norm_eps, num_buckets,
                                   max_distance, hd, stream)
    return int(load().tsfm_bolt_forecast_horizon(ctypes.byref(a)))


def bolt_forecast_horizon_args(out, inputs, horizon, reg, dec_start, rel_table, enc_layers, enc_final_norm,
                               dec_layers, dec_final_norm, input_embed, output_embed, d, nh, d_ff, eps,
                               quantile_levels, prediction_length, context_length, patch=16, norm_eps=1e-5,
                               num_buckets=32, max_distance=128, hd=64, stream=None) -> BoltHorizonArgs:
    """The argument block of bolt_forecast_horizon, built once for repeated calls (it keeps what it
    points to alive)."""
    import numpy as np

    b, t_in = int(inputs.shape[0]), int(inputs.shape[1])
    levels = np.ascontiguousarray(quantile_levels, np.float32)
    m = bolt_forward_args(enc_layers, dec_layers, None, None, reg, dec_start, rel_table, enc_final_norm, dec_final_norm,
                          input_embed, output_embed, None, b, 0, d, nh, hd, d_ff, eps, num_buckets, max_distance, False,
                          True, stream)
    if not _is_device(inputs):  # host inputs and out, device weights: TSFM_FORECAST_HOST_IO
        m.flags |= FORECAST_HOST_IO
    a = BoltHorizonArgs(model=m, inputs=_ptr(inputs), t_in=t_in, horizon=horizon, patch=patch,
                        prediction_length=prediction_length, context_length=context_length, n_quantiles=levels.size,
                        quantile_levels=levels.ctypes.data, norm_eps=norm_eps, out=_ptr(out))
    a._keep = (m._keep, levels, inputs, out)
    return a


def weight_register(w) -> Optional[int]:
    """``tsfm_weight_register`` (Backend.register_weight): device copy of a C-contiguous f32 array;
    the handle, or None on failure."""
    n = int(w.numel()) if hasattr(w, "numel") else int(w.size)
    h = load().tsfm_weight_register(_ptr(w), n)
    return h or None


def weight_release(handle: Optional[int]) -> None:
    load().tsfm_weight_release(handle)


def sgemm_nt(m: int, n: int, k: int, alpha: float, a, lda: int, b, ldb: int, c, ldc: int, b_buf=None) -> int:
    """``tsfm_sgemm_nt`` (Backend.sgemm_nt): c[m, n] = alpha * a[m, k] b[n, k]^T with leading
    dimensions, host arrays; ``b_buf`` a handle from :func:`weight_register` (then ``b`` is unused)."""
    return int(load().tsfm_sgemm_nt(m, n, k, alpha, _ptr(a), lda, _ptr(b), ldb, _ptr(c), ldc, b_buf))


def sgemm_nn(m: int, n: int, k: int, a, lda: int, b, ldb: int, c, ldc: int, b_buf=None) -> int:
    """``tsfm_sgemm_nn`` (Backend.sgemm_nn): c[m, n] = a[m, k] b[k, n] with leading dimensions, host
    arrays; ``b_buf`` a handle from :func:`weight_register` holding b as [k][ldb] (then ``b`` is
    unused)."""
    return int(load().tsfm_sgemm_nn(m, n, k, _ptr(a), lda, _ptr(b), ldb, _ptr(c), ldc, b_buf))


def linear(y, x, rows: int, w, out: int, inp: int, w_buf=None) -> int:
    """nn.linear without bias through the backend seam (src/core/nn.zig:270-293): y (rows, out) =
    x (rows, inp) w (out, inp)^T."""
    return sgemm_nt(rows, out, inp, 1.0, x, inp, w, inp, y, out, w_buf)


# ---------------------------------------------------------------------------------------------
# KV cache (no counterpart in the reference: Timestral's blockDecode re-encodes the whole context
# every block, src/timestral/forecaster.zig:423-563).


class KvCache:
    """``tsfm_kv_*``: a device K/V cache of ``capacity`` tokens for every (series, head), bf16 or
    f16. ``append`` adds the K/V of new tokens; ``attend`` runs causal attention of queries at
    positions ``q_pos0..`` over the cached keys. Arrays follow the (B, tokens, H*D) layout with
    token/batch strides in elements; device tensors make the calls asynchronous on the given (or
    current) stream, numpy arrays make them synchronous."""

    def __init__(self, dtype: int, batch: int, heads: int, capacity: int, head_dim: int = 64):
        self.dtype, self.batch, self.heads, self.head_dim = dtype, batch, heads, head_dim
        h = ctypes.c_void_p()
        rc = load().tsfm_kv_create(ctypes.byref(h), dtype, batch, heads, head_dim, capacity)
        if rc != OK:
            raise TsfmError(rc, last_error())
        self._h = h

    def _check(self, rc: int) -> None:
        if rc != OK:
            raise TsfmError(rc, last_error())

    @property
    def handle(self) -> int:
        return int(self._h.value or 0)

    def __len__(self) -> int:
        return int(load().tsfm_kv_len(self._h))

    def append(self, k, v, n_new: int, k_tok: int, k_batch: int, v_tok: int, v_batch: int, stream=None) -> None:
        device = _is_device(k)
        self._check(load().tsfm_kv_append(self._h, _ptr(k), k_tok, k_batch, _ptr(v), v_tok, v_batch, n_new,
                                          DEVICE_PTRS if device else 0, _stream_of(k, stream) if device else None))

    def attend(self, q, o, n_q: int, q_pos0: int, scale: float, q_tok: int, q_batch: int, o_tok: int, o_batch: int,
               stream=None) -> None:
        device = _is_device(q)
        self._check(load().tsfm_kv_attend(self._h, _ptr(q), q_tok, q_batch, _ptr(o), o_tok, o_batch, n_q, q_pos0,
                                          float(scale), DEVICE_PTRS if device else 0,
                                          _stream_of(q, stream) if device else None))

    def append_attend(self, k, v, q, o, n_new: int, scale: float, k_tok: int, k_batch: int, v_tok: int, v_batch: int,
                      q_tok: int, q_batch: int, o_tok: int, o_batch: int, stream=None) -> None:
        """One decode block: ``append`` of the new tokens' k/v, then ``attend`` of their queries at
        positions ``len(self)..`` (one launch for device tensors, n_new == 32 and len(self) a multiple
        of 32)."""
        device = _is_device(q)
        self._check(load().tsfm_kv_append_attend(self._h, _ptr(k), k_tok, k_batch, _ptr(v), v_tok, v_batch, _ptr(q),
                                                 q_tok, q_batch, _ptr(o), o_tok, o_batch, n_new, float(scale),
                                                 DEVICE_PTRS if device else 0,
                                                 _stream_of(q, stream) if device else None))

    def truncate(self, length: int) -> None:
        self._check(load().tsfm_kv_truncate(self._h, length))

    def reset(self) -> None:
        self._check(load().tsfm_kv_reset(self._h))

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            load().tsfm_kv_free(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self) -> "KvCache":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


# ---- Timestral forecast -------------------------------------------------------------------------


def timestral_forecast_args(out, inputs, observed, model: dict, batch: int, variates: int, length: int, horizon: int,
                            max_context: int = 0, per_shot: int = 32, cap_k: float = 1e4, extreme: float = 1e30,
                            symmetric: bool = True, clip_nonnegative: bool = True, kv_cache: bool = True,
                            attn_bf16: bool = False, past=None, known=None, stream=None) -> "TimestralForecastArgs":
    """``tsfm_timestral_forecast_args``: inputs, observed, covariates and out as device tensors, or
    all as host numpy arrays (TSFM_FORECAST_HOST_IO: synchronous). `model` holds the config and device
    weights (keys as in the reference checkpoint's layout: patch_proj/head ResBlocks, layers with
    attns [is_time, norm, qkv (permuted), out, gate] and mlp_norm/w12/w3, forecast_query, out_norm,
    knots (host float64 array)). attn_bf16 sets TSFM_TIMESTRAL_BF16_ATTN (time attention on the bf16
    matrix cores over a bf16 K/V cache). past (batch, n_past, length) and known (batch, n_known,
    length + horizon) are numeric covariates, NaN = missing (forecaster.zig:36-46). The returned block
    keeps references to what it points at."""
    import numpy as np

    layers = (TimestralLayer * max(1, len(model["layers"])))()
    for i, ly in enumerate(model["layers"]):
        layers[i].n_attn = len(ly["attns"])
        for j, at in enumerate(ly["attns"]):
            layers[i].attn[j] = TimestralAttn(int(at["is_time"]), _ptr(at["norm"]), _ptr(at["qkv"]), _ptr(at["out"]),
                                              _ptr(at.get("gate")))
        layers[i].mlp_norm, layers[i].w12, layers[i].w3 = _ptr(ly["mlp_norm"]), _ptr(ly["w12"]), _ptr(ly["w3"])
    knots = np.ascontiguousarray(model["knots"], np.float64)
    m = TimestralModel(patch=model["ps"], d_model=model["d"], heads=model["nh"], head_dim=64, mlp_hidden=model["hid"],
                       n_layers=len(model["layers"]), n_quantiles=model["q"], block_size=model["block_size"],
                       context_length=model["context_length"], rope_dim=model["rope_dim"],
                       use_asinh=int(model["use_asinh"]), attend_missing=int(model["attend_missing"]),
                       covariate_enabled=int(model.get("covariate_enabled", True)),
                       rope_theta=model["rope_theta"], norm_eps=model["norm_eps"], minimum_scale=model["minimum_scale"],
                       quantile_width_factor=model["width_factor"], quantile_knots=knots.ctypes.data,
                       patch_proj=_resblock(model["patch_proj"], act=1), head=_resblock(model["head"], act=1),
                       forecast_query=_ptr(model["forecast_query"]), out_norm=_ptr(model["out_norm"]), layers=layers)
    a = TimestralForecastArgs(model=m, inputs=_ptr(inputs), observed=_ptr(observed), batch=batch, variates=variates,
                              len=length, horizon=horizon, max_context=max_context, per_shot_patches=per_shot,
                              quantile_real_cap_k=cap_k, extreme_value_threshold=extreme,
                              symmetric_averaging=int(symmetric), clip_nonnegative=int(clip_nonnegative),
                              kv_cache=int(kv_cache),
                              flags=DEVICE_PTRS | (TIMESTRAL_BF16_ATTN if attn_bf16 else 0) |
                              (0 if _is_device(inputs) else FORECAST_HOST_IO),
                              out=_ptr(out), stream=_stream_of(out, stream), past=_ptr(past), known=_ptr(known),
                              n_past=0 if past is None else int(past.shape[1]),
                              n_known=0 if known is None else int(known.shape[1]))
    a._keep = (layers, knots, model, inputs, observed, out, past, known)
    return a


class CategoricalArgs(ctypes.Structure):
    """``tsfm_categorical_args`` (include/tsfm_attn.h)."""
    _fields_ = [
        ("out", ctypes.c_void_p),
        ("out_rows", ctypes.c_int32),
        ("row0", ctypes.c_int32),
        ("codes", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("n_cat", ctypes.c_int32),
        ("len", ctypes.c_int64),
        ("inputs", ctypes.c_void_p),
        ("observed", ctypes.c_void_p),
        ("variates", ctypes.c_int32),
        ("t", ctypes.c_int64),
        ("max_context", ctypes.c_int64),
    ]


def timestral_encode_categorical(codes, inputs, observed, max_context: int, out=None, row0: int = 0) -> np.ndarray:
    """Categorical covariates as numeric rows (forecaster.zig:86-103, 201-301), on the host:
    codes (batch, n_cat, len) f64 (NaN = missing, len = t for past codes, t + horizon for known
    ones), inputs / observed (batch, variates, t). Returns out (batch, out_rows, len) f32 with the
    encoded rows at row0 .. row0 + n_cat - 1 (a new (batch, n_cat, len) array when out is None).
    Raises ValueError with the library's message on an invalid request."""
    codes = np.ascontiguousarray(codes, np.float64)
    inputs = np.ascontiguousarray(inputs, np.float32)
    observed = np.ascontiguousarray(observed, np.uint8)
    b, c, n = codes.shape
    if out is None:
        out = np.zeros((b, c, n), np.float32)
    if out.dtype != np.float32 or not out.flags.c_contiguous or out.ndim != 3 or out.shape[0] != b or out.shape[2] != n:
        raise ValueError("out must be a C-contiguous (batch, rows, len) float32 array")
    a = CategoricalArgs(out=out.ctypes.data, out_rows=out.shape[1], row0=row0, codes=codes.ctypes.data, batch=b,
                        n_cat=c, len=n, inputs=inputs.ctypes.data, observed=observed.ctypes.data,
                        variates=inputs.shape[1], t=inputs.shape[2], max_context=max_context)
    rc = int(load().tsfm_timestral_encode_categorical(ctypes.byref(a)))
    if rc != OK:
        raise ValueError(last_error())
    return out


def timestral_forecast(out, inputs, observed, model: dict, batch: int, variates: int, length: int, horizon: int,
                       cat_past=None, cat_known=None, **kw) -> int:
    """Timestral forecaster.forecast (src/timestral/forecaster.zig:57-180) on device tensors: inputs
    (batch, variates, length) f32, observed (same) uint8, out (batch, variates, horizon, q);
    optional numeric covariates past= / known= (see timestral_forecast_args) and categorical codes
    cat_past= (batch, n, length) / cat_known= (batch, n, length + horizon) as float64 host arrays,
    encoded on the host (timestral_encode_categorical) and appended after the numeric rows of each
    series, as the reference does. Returns the ABI code."""
    if cat_past is not None or cat_known is not None:
        import torch

        host = lambda a: a if isinstance(a, np.ndarray) else a.detach().cpu().numpy()  # noqa: E731
        device = _is_device(inputs)
        x = host(inputs).reshape(batch, variates, length)
        ob = host(observed).reshape(batch, variates, length)
        window = int(kw.get("max_context", 0) or model["context_length"])
        for key, codes, n in (("past", cat_past, length), ("known", cat_known, length + horizon)):
            if codes is None:
                continue
            codes = np.asarray(codes, np.float64)
            numeric = kw.get(key)
            n_num = 0 if numeric is None else int(numeric.shape[1])
            rows = np.zeros((batch, n_num + codes.shape[1], n), np.float32)
            if numeric is not None:
                rows[:, :n_num] = host(numeric)
            timestral_encode_categorical(codes, x, ob, window, out=rows, row0=n_num)
            kw[key] = torch.from_numpy(rows).to(out.device) if device else rows
    args = timestral_forecast_args(out, inputs, observed, model, batch, variates, length, horizon, **kw)
    return int(load().tsfm_timestral_forecast(ctypes.byref(args)))

