"""ctypes wrapper of the CPU oracle (oracle/liboracle_l*.so) for the tests and the CPU baseline.

Test infrastructure: results are checked against it; it is never the thing measured or shipped.
"""
import ctypes

import numpy as np

ORC_FULL, ORC_KEYS_ADDITIVE, ORC_CAUSAL, ORC_CAUSAL_KEYS, ORC_FULL_KEYS = range(5)

_sz = ctypes.c_size_t
_vp = ctypes.c_void_p
_f = ctypes.c_float


def ptr(a):
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous numpy arrays"
    return a.ctypes.data


LAYER_FIELDS = ("time_norm", "time_q", "time_k", "time_v", "time_o", "group_norm", "group_v", "group_o", "mlp_norm",
                "mlp_wi", "mlp_wo")


class Chronos2Layer(ctypes.Structure):
    """orc_chronos2_layer (oracle/tsfm_oracle.h)."""

    _fields_ = [(f, _vp) for f in LAYER_FIELDS]


RESBLOCK_FIELDS = ("hidden_w", "hidden_b", "output_w", "output_b", "residual_w", "residual_b")


class OrcResblock(ctypes.Structure):
    """orc_resblock (oracle/tsfm_oracle.h)."""

    _fields_ = [(f, _vp) for f in RESBLOCK_FIELDS] + [("in_", _sz), ("hid", _sz), ("out", _sz)]


def resblock_struct(rb):
    """rb: dict of the RESBLOCK_FIELDS arrays (weights (out, in) layout)."""
    st = OrcResblock()
    for f in RESBLOCK_FIELDS:
        setattr(st, f, ptr(rb[f]))
    st.hid, st.in_ = rb["hidden_w"].shape
    st.out = rb["output_w"].shape[0]
    return st


BOLT_ENC_FIELDS = ("attn_norm", "q", "k", "v", "o", "ffn_norm", "wi", "wo")
BOLT_DEC_FIELDS = ("self_norm", "self_v", "self_o", "cross_norm", "cross_q", "cross_k", "cross_v", "cross_o",
                   "ffn_norm", "wi", "wo")


class BoltEncLayer(ctypes.Structure):
    _fields_ = [(f, _vp) for f in BOLT_ENC_FIELDS]


class BoltDecLayer(ctypes.Structure):
    _fields_ = [(f, _vp) for f in BOLT_DEC_FIELDS]


class OrcBoltModel(ctypes.Structure):
    _fields_ = [("reg", ctypes.c_void_p), ("dec_start", ctypes.c_void_p), ("rel_table", ctypes.c_void_p),
                ("num_buckets", ctypes.c_uint32), ("max_distance", ctypes.c_uint32), ("d", ctypes.c_size_t),
                ("nh", ctypes.c_size_t), ("hd", ctypes.c_size_t), ("d_ff", ctypes.c_size_t),
                ("enc", ctypes.POINTER(BoltEncLayer)), ("n_enc", ctypes.c_size_t), ("enc_final_norm", ctypes.c_void_p),
                ("dec", ctypes.POINTER(BoltDecLayer)), ("n_dec", ctypes.c_size_t), ("dec_final_norm", ctypes.c_void_p),
                ("eps", ctypes.c_float), ("input_embed", ctypes.POINTER(OrcResblock)),
                ("output_embed", ctypes.POINTER(OrcResblock))]


def bolt_model_struct(w):
    """OrcBoltModel over a dict with reg, dec_start, rel_table, enc, dec, enc_final_norm,
    dec_final_norm, ie, oe (host arrays) and d_model, heads, d_ff, eps, buckets, max_distance. The
    struct keeps what it points to alive."""
    enc, dec = w["enc"], w["dec"]
    ea = (BoltEncLayer * max(1, len(enc)))()
    for i, ly in enumerate(enc):
        for f in BOLT_ENC_FIELDS:
            setattr(ea[i], f, ptr(ly[f]))
    da = (BoltDecLayer * max(1, len(dec)))()
    for i, ly in enumerate(dec):
        for f in BOLT_DEC_FIELDS:
            setattr(da[i], f, ptr(ly[f]))
    ie, oe = resblock_struct(w["ie"]), resblock_struct(w["oe"])
    m = OrcBoltModel(reg=ptr(w["reg"]), dec_start=ptr(w["dec_start"]), rel_table=ptr(w["rel_table"]),
                     num_buckets=w["buckets"], max_distance=w["max_distance"], d=w["d_model"], nh=w["heads"], hd=64,
                     d_ff=w["d_ff"], enc=ea, n_enc=len(enc), enc_final_norm=ptr(w["enc_final_norm"]), dec=da,
                     n_dec=len(dec), dec_final_norm=ptr(w["dec_final_norm"]), eps=w["eps"],
                     input_embed=ctypes.pointer(ie), output_embed=ctypes.pointer(oe))
    m._keep = (ea, da, ie, oe, w)
    return m


class TimestralAttn(ctypes.Structure):
    """orc_timestral_attn (oracle/tsfm_oracle.h)."""

    _fields_ = [("is_time", ctypes.c_int), ("norm", _vp), ("qkv", _vp), ("out", _vp), ("gate", _vp)]


class TimestralLayer(ctypes.Structure):
    _fields_ = [("n_attn", ctypes.c_int), ("attn", TimestralAttn * 2), ("mlp_norm", _vp), ("w12", _vp), ("w3", _vp)]


class TimestralModel(ctypes.Structure):
    _fields_ = [(f, _sz) for f in ("ps", "d", "nh", "hd", "hid", "n_layers", "q", "median", "block_size",
                                   "context_length", "rope_dim")] + \
               [("rope_theta", _f), ("norm_eps", _f), ("quantile_width_factor", _f), ("minimum_scale", ctypes.c_double),
                ("use_asinh", ctypes.c_int), ("attend_missing", ctypes.c_int), ("knots", _vp),
                ("patch_proj", OrcResblock), ("head", OrcResblock), ("forecast_query", _vp), ("out_norm", _vp),
                ("layers", ctypes.POINTER(TimestralLayer))]


def timestral_model_struct(m):
    """orc_timestral_model from a model dict (tests/_ref.py timestral_model); the returned struct keeps
    references to everything it points at."""
    layers = (TimestralLayer * max(1, len(m["layers"])))()
    for i, ly in enumerate(m["layers"]):
        layers[i].n_attn = len(ly["attns"])
        for j, a in enumerate(ly["attns"]):
            layers[i].attn[j] = TimestralAttn(int(a["is_time"]), ptr(a["norm"]), ptr(a["qkv"]), ptr(a["out"]),
                                              ptr(a.get("gate")))
        layers[i].mlp_norm, layers[i].w12, layers[i].w3 = ptr(ly["mlp_norm"]), ptr(ly["w12"]), ptr(ly["w3"])
    st = TimestralModel(ps=m["ps"], d=m["d"], nh=m["nh"], hd=64, hid=m["hid"], n_layers=len(m["layers"]), q=m["q"],
                        median=m["median"], block_size=m["block_size"], context_length=m["context_length"],
                        rope_dim=m["rope_dim"], rope_theta=m["rope_theta"], norm_eps=m["norm_eps"],
                        quantile_width_factor=m["width_factor"], minimum_scale=m["minimum_scale"],
                        use_asinh=int(m["use_asinh"]), attend_missing=int(m["attend_missing"]), knots=ptr(m["knots"]),
                        patch_proj=resblock_struct(m["patch_proj"]), head=resblock_struct(m["head"]),
                        forecast_query=ptr(m["forecast_query"]), out_norm=ptr(m["out_norm"]), layers=layers)
    st._keep = (layers, m)
    return st


class Oracle:
    def __init__(self, path):
        self.path = str(path)
        L = self.lib = ctypes.CDLL(self.path)
        L.orc_lanes.restype = ctypes.c_int
        L.orc_exp_vec.argtypes = [_f]
        L.orc_exp_vec.restype = _f
        L.orc_gemm_nt.argtypes = [_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _f]
        L.orc_gemm_nn.argtypes = [_vp, _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz]
        L.orc_linear.argtypes = [_sz, _vp, _vp, _sz, _vp, _sz, _sz, _vp]
        L.orc_rms_norm.argtypes = [_sz, _vp, _vp, _sz, _sz, _vp, _f]
        L.orc_relu.argtypes = [_vp, _sz]
        L.orc_resblock_relu.argtypes = [_sz, _vp, _vp, _sz, ctypes.POINTER(OrcResblock)]
        L.orc_bolt_forecast.argtypes = [_sz, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _f, _vp, _vp, _vp, ctypes.c_uint32,
                                        ctypes.c_uint32, _sz, _sz, _sz, _sz, ctypes.POINTER(BoltEncLayer), _sz, _vp,
                                        ctypes.POINTER(BoltDecLayer), _sz, _vp, _f, ctypes.POINTER(OrcResblock),
                                        ctypes.POINTER(OrcResblock)]
        L.orc_bolt_model_forward.argtypes = [_sz, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_uint32, ctypes.c_uint32, _sz,
                                             _sz, _sz, _sz, _sz, _sz, ctypes.POINTER(BoltEncLayer), _sz, _vp,
                                             ctypes.POINTER(BoltDecLayer), _sz, _vp, _f, ctypes.POINTER(OrcResblock),
                                             ctypes.POINTER(OrcResblock)]
        L.orc_chronos2_model_forward.argtypes = [_sz, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz,
                                                 ctypes.POINTER(Chronos2Layer), _vp, _f, _vp, _vp, _f,
                                                 ctypes.POINTER(OrcResblock), ctypes.POINTER(OrcResblock)]
        L.orc_chronos2_forecast.argtypes = [_sz, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _f, ctypes.c_int, _vp, _sz,
                                            _sz, _sz, _sz, _sz, ctypes.POINTER(Chronos2Layer), _vp, _f, _vp, _vp, _f,
                                            ctypes.POINTER(OrcResblock), ctypes.POINTER(OrcResblock)]
        L.orc_chronos2_encode.argtypes = [_sz, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, ctypes.POINTER(Chronos2Layer),
                                          _vp, _f, _vp, _vp, _f]
        L.orc_softmax.argtypes = [_vp, _sz]
        L.orc_dot.argtypes = [_vp, _vp, _sz]
        L.orc_dot.restype = _f
        L.orc_rope_half.argtypes = [_vp, _vp, _vp, _sz]
        L.orc_mask_pick.argtypes = [ctypes.c_int] * 3
        L.orc_mask_pick.restype = ctypes.c_int
        L.orc_masked_softmax.argtypes = [ctypes.c_int, _vp, _sz, _vp]
        L.orc_self_attend.argtypes = [ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _f, _vp, _vp]
        L.orc_reference_attend_f64.argtypes = [ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _sz, _sz, ctypes.c_double, _vp, _vp]
        L.orc_relative_bucket.argtypes = [ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_relative_bucket.restype = ctypes.c_uint32
        L.orc_position_bias.argtypes = [_vp, _vp, _sz, _sz, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_bolt_self_attention.argtypes = [_sz, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int, _sz, _sz, _sz, _sz, _sz]
        L.orc_bolt_cross_attention.argtypes = [_sz, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz]
        L.orc_chronos2_rope_tables.argtypes = [_vp, _vp, _sz, _sz, _f]
        L.orc_chronos2_rope.argtypes = [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz]
        L.orc_chronos2_time_attention.argtypes = [_sz, _vp, _vp, _vp, _vp, _vp, ctypes.c_int, _sz, _sz, _sz, _sz, _sz, _f]
        L.orc_timestral_key_valid.argtypes = [_vp, _vp, _vp, _sz, _sz, _sz, _sz, ctypes.c_int]
        L.orc_timestral_key_valid.restype = ctypes.c_int
        L.orc_timestral_rope_tables.argtypes = [_vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _f, _vp]
        L.orc_timestral_rope.argtypes = [_sz, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz]
        L.orc_timestral_time_attention.argtypes = [_sz, _vp, _vp, _vp, ctypes.c_int, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz]
        L.orc_timestral_variate_attention.argtypes = [_sz, _vp, _vp, _vp, _vp, ctypes.c_int, _sz, _sz, _sz, _sz, _sz, _sz,
                                                      _sz]
        L.orc_mul_sigmoid.argtypes = [_vp, _vp, _vp, _sz]
        L.orc_silu_in_place.argtypes = [_vp, _sz]
        L.orc_mul_silu.argtypes = [_vp, _vp, _vp, _sz]
        L.orc_softplus.argtypes = [_f]
        L.orc_softplus.restype = _f
        L.orc_clamp_nonfinite.argtypes = [_vp, _sz]
        L.orc_resblock_silu.argtypes = [_sz, _vp, _vp, _sz, ctypes.POINTER(OrcResblock)]
        L.orc_timestral_patch_stats.argtypes = [_sz, _vp, _vp, _vp, _vp, _sz, _sz, _sz, ctypes.c_double]
        L.orc_timestral_predict_block.argtypes = [_sz, _vp, ctypes.POINTER(TimestralModel), _vp, _vp, _sz, _sz, _sz, _sz]
        L.orc_timestral_refine_block.argtypes = [_vp, ctypes.POINTER(TimestralModel), _vp, _vp, _sz, _sz, _sz]
        L.orc_timestral_forecast.argtypes = [_sz, _vp, ctypes.POINTER(TimestralModel), _vp, _vp, _sz, _sz, _sz, _sz, _sz,
                                             _sz, _f, _f, ctypes.c_int, ctypes.c_int]
        L.orc_timestral_forecast.restype = ctypes.c_int
        L.orc_timestral_predict_block_cov.argtypes = [_sz, _vp, ctypes.POINTER(TimestralModel), _vp, _vp, _sz, _sz, _sz,
                                                      _sz, _vp, _vp, _vp]
        L.orc_timestral_forecast_cov.argtypes = [_sz, _vp, ctypes.POINTER(TimestralModel), _vp, _vp, _sz, _sz, _sz, _sz,
                                                 _vp, _sz, _vp, _sz, _sz, _sz, _f, _f, ctypes.c_int, ctypes.c_int]
        L.orc_timestral_forecast_cov.restype = ctypes.c_int
        L.orc_timestral_encode_categorical.argtypes = [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _sz, _sz, _sz]
        L.orc_timestral_encode_categorical.restype = None
        L.orc_quantile_linear.argtypes = [_vp, _sz, _f]
        L.orc_quantile_linear.restype = _f
        L.orc_bolt_forecast_horizon.argtypes = [_sz, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _sz, _f,
                                                ctypes.POINTER(OrcBoltModel)]
        L.orc_batched_self_attend.argtypes = [_sz, ctypes.c_int, _vp, _sz, _sz, _vp, _sz, _sz, _vp, _sz, _sz, _vp, _sz,
                                              _sz, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _f]

    @property
    def lanes(self):
        return self.lib.orc_lanes()

    # ---- nn.zig ----
    def exp_vec(self, x):
        return np.float32(self.lib.orc_exp_vec(float(x)))

    def gemm_nt(self, c, ldc, a, lda, b, ldb, m, n, k, alpha):
        self.lib.orc_gemm_nt(ptr(c), ldc, ptr(a), lda, ptr(b), ldb, m, n, k, alpha)

    def linear(self, threads, y, x, rows, w, out, inp, bias=None):
        """nn.linear: y (rows, out) = x (rows, inp) w (out, inp)^T (+ bias)."""
        self.lib.orc_linear(threads, ptr(y), ptr(x), rows, ptr(w), out, inp, ptr(bias))

    def rms_norm(self, threads, out, x, rows, dim, scale, eps):
        self.lib.orc_rms_norm(threads, ptr(out), ptr(x), rows, dim, ptr(scale), eps)

    def relu(self, x):
        self.lib.orc_relu(ptr(x), x.size)

    def chronos2_encode(self, threads, x, key_valid, b, seq, d, nh, hd, d_ff, layers, final_norm, eps, cos_t, sin_t,
                        scale):
        """x (b*seq, d) in place; layers: list of dicts of the LAYER_FIELDS arrays."""
        arr = (Chronos2Layer * max(1, len(layers)))()
        for i, ly in enumerate(layers):
            for f in LAYER_FIELDS:
                setattr(arr[i], f, ptr(ly[f]))
        self.lib.orc_chronos2_encode(threads, ptr(x), ptr(key_valid), b, seq, d, nh, hd, d_ff, len(layers), arr,
                                     ptr(final_norm), eps, ptr(cos_t), ptr(sin_t), scale)

    def resblock_relu(self, threads, y, x, rows, rb):
        st = resblock_struct(rb)
        self.lib.orc_resblock_relu(threads, ptr(y), ptr(x), rows, ctypes.byref(st))

    def chronos2_model_forward(self, threads, raw, feats, fut_feats, ctx_valid, reg, b, n_ctx, n_out, d, nh, hd, d_ff,
                               layers, final_norm, eps, cos_t, sin_t, scale, input_embed, output_embed):
        arr = (Chronos2Layer * max(1, len(layers)))()
        for i, ly in enumerate(layers):
            for f in LAYER_FIELDS:
                setattr(arr[i], f, ptr(ly[f]))
        ie, oe = resblock_struct(input_embed), resblock_struct(output_embed)
        self.lib.orc_chronos2_model_forward(threads, ptr(raw), ptr(feats), ptr(fut_feats), ptr(ctx_valid), ptr(reg), b,
                                            n_ctx, n_out, d, nh, hd, d_ff, len(layers), arr, ptr(final_norm), eps,
                                            ptr(cos_t), ptr(sin_t), scale, ctypes.byref(ie), ctypes.byref(oe))

    def chronos2_forecast(self, threads, out, inputs, stride, start, length, n, ps, horizon, time_scale, arcsinh, reg,
                          d, nh, hd, d_ff, layers, final_norm, eps, cos_t, sin_t, scale, input_embed, output_embed):
        arr = (Chronos2Layer * max(1, len(layers)))()
        for i, ly in enumerate(layers):
            for f in LAYER_FIELDS:
                setattr(arr[i], f, ptr(ly[f]))
        ie, oe = resblock_struct(input_embed), resblock_struct(output_embed)
        self.lib.orc_chronos2_forecast(threads, ptr(out), ptr(inputs), stride, start, length, n, ps, horizon,
                                       time_scale, int(bool(arcsinh)), ptr(reg), d, nh, hd, d_ff, len(layers), arr,
                                       ptr(final_norm), eps, ptr(cos_t), ptr(sin_t), scale, ctypes.byref(ie),
                                       ctypes.byref(oe))

    def bolt_model_forward(self, threads, raw, feats, patch_valid, reg, dec_start, rel_table, buckets, max_distance,
                           b, n_patch, d, nh, hd, d_ff, enc, enc_final_norm, dec, dec_final_norm, eps, input_embed,
                           output_embed):
        ea = (BoltEncLayer * max(1, len(enc)))()
        for i, ly in enumerate(enc):
            for f in BOLT_ENC_FIELDS:
                setattr(ea[i], f, ptr(ly[f]))
        da = (BoltDecLayer * max(1, len(dec)))()
        for i, ly in enumerate(dec):
            for f in BOLT_DEC_FIELDS:
                setattr(da[i], f, ptr(ly[f]))
        ie, oe = resblock_struct(input_embed), resblock_struct(output_embed)
        self.lib.orc_bolt_model_forward(threads, ptr(raw), ptr(feats), ptr(patch_valid), ptr(reg), ptr(dec_start),
                                        ptr(rel_table), buckets, max_distance, b, n_patch, d, nh, hd, d_ff, ea, len(enc),
                                        ptr(enc_final_norm), da, len(dec), ptr(dec_final_norm), eps, ctypes.byref(ie),
                                        ctypes.byref(oe))

    def bolt_forecast(self, threads, out, ctx, stride, offset, length, n, ps, norm_eps, reg, dec_start, rel_table,
                      buckets, max_distance, d, nh, hd, d_ff, enc, enc_final_norm, dec, dec_final_norm, eps,
                      input_embed, output_embed):
        ea = (BoltEncLayer * max(1, len(enc)))()
        for i, ly in enumerate(enc):
            for f in BOLT_ENC_FIELDS:
                setattr(ea[i], f, ptr(ly[f]))
        da = (BoltDecLayer * max(1, len(dec)))()
        for i, ly in enumerate(dec):
            for f in BOLT_DEC_FIELDS:
                setattr(da[i], f, ptr(ly[f]))
        ie, oe = resblock_struct(input_embed), resblock_struct(output_embed)
        self.lib.orc_bolt_forecast(threads, ptr(out), ptr(ctx), stride, offset, length, n, ps, norm_eps, ptr(reg),
                                   ptr(dec_start), ptr(rel_table), buckets, max_distance, d, nh, hd, d_ff, ea, len(enc),
                                   ptr(enc_final_norm), da, len(dec), ptr(dec_final_norm), eps, ctypes.byref(ie),
                                   ctypes.byref(oe))

    def quantile_linear(self, sorted_vals, level):
        a = np.ascontiguousarray(sorted_vals, np.float32)
        return np.float32(self.lib.orc_quantile_linear(ptr(a), a.size, level))

    def bolt_forecast_horizon(self, threads, inputs, horizon, w, P, max_ctx, levels, ps=16, norm_eps=1e-5):
        """(b, horizon, q) of forecaster.forecast for inputs (b, t_in); w as bolt_model_struct takes."""
        x = np.ascontiguousarray(inputs, np.float32)
        b, t_in = x.shape
        lv = np.ascontiguousarray(levels, np.float32)
        out = np.zeros((b, horizon, lv.size), np.float32)
        m = bolt_model_struct(w)
        self.lib.orc_bolt_forecast_horizon(threads, ptr(out), ptr(x), b, t_in, horizon, ps, P, max_ctx, ptr(lv),
                                           lv.size, norm_eps, ctypes.byref(m))
        return out

    def gemm_nn(self, c, ldc, a, lda, b, ldb, m, n, k):
        self.lib.orc_gemm_nn(ptr(c), ldc, ptr(a), lda, ptr(b), ldb, m, n, k)

    def softmax(self, row):
        self.lib.orc_softmax(ptr(row), row.size)

    def dot(self, a, b):
        return np.float32(self.lib.orc_dot(ptr(a), ptr(b), min(a.size, b.size)))

    def rope_half(self, x, cos_t, sin_t, half):
        self.lib.orc_rope_half(ptr(x), ptr(cos_t), ptr(sin_t), half)

    # ---- attn.zig ----
    def mask_pick(self, causal, all_valid, additive):
        return self.lib.orc_mask_pick(int(causal), int(all_valid), int(additive))

    def masked_softmax(self, mask, scores, n, key_valid):
        self.lib.orc_masked_softmax(mask, ptr(scores), n, ptr(key_valid))

    def self_attend(self, mask, q, k, v, o, st, n, hd, scale, key_valid=None, bias=None):
        scores = np.empty(max(n * n, 1), np.float32)
        st_arr = (ctypes.c_size_t * 4)(*st)
        self.lib.orc_self_attend(mask, ptr(scores), ptr(q), ptr(k), ptr(v), ptr(o), st_arr, n, hd, scale,
                                 ptr(key_valid), ptr(bias))

    def reference_attend_f64(self, mask, q, k, v, st, n, hd, scale, key_valid=None, bias=None):
        o = np.empty(n * hd, np.float64)
        st_arr = (ctypes.c_size_t * 4)(*st)
        kv = key_valid if key_valid is not None else np.ones(n, np.uint8)
        self.lib.orc_reference_attend_f64(mask, ptr(o), ptr(q), ptr(k), ptr(v), st_arr, n, hd, scale, ptr(kv), ptr(bias))
        return o.reshape(n, hd)

    # ---- families ----
    def relative_bucket(self, rel, nb, maxd):
        return self.lib.orc_relative_bucket(rel, nb, maxd)

    def position_bias(self, table, seq, nh, nb, maxd):
        out = np.empty(nh * seq * seq, np.float32)
        self.lib.orc_position_bias(ptr(out), ptr(table), seq, nh, nb, maxd)
        return out

    def bolt_self_attention(self, threads, q, k, v, o, bias, key_valid, keys_all_valid, nb, seq, inner, nh, hd):
        self.lib.orc_bolt_self_attention(threads, ptr(q), ptr(k), ptr(v), ptr(o), ptr(bias), ptr(key_valid),
                                         int(keys_all_valid), nb, seq, inner, nh, hd)

    def bolt_cross_attention(self, threads, q, k, v, o, key_valid, nb, seq, inner, nh, hd):
        self.lib.orc_bolt_cross_attention(threads, ptr(q), ptr(k), ptr(v), ptr(o), ptr(key_valid), nb, seq, inner, nh, hd)

    def chronos2_rope_tables(self, seq, hd, theta=10000.0):
        c = np.empty(seq * (hd // 2), np.float32)
        s = np.empty_like(c)
        self.lib.orc_chronos2_rope_tables(ptr(c), ptr(s), seq, hd, theta)
        return c, s

    def chronos2_rope(self, q, k, cos_t, sin_t, rows, seq, d, nh, hd):
        self.lib.orc_chronos2_rope(ptr(q), ptr(k), ptr(cos_t), ptr(sin_t), rows, seq, d, nh, hd)

    def chronos2_time_attention(self, threads, q, k, v, o, key_valid, keys_all_valid, b, seq, d, nh, hd, scale):
        self.lib.orc_chronos2_time_attention(threads, ptr(q), ptr(k), ptr(v), ptr(o), ptr(key_valid),
                                             int(keys_all_valid), b, seq, d, nh, hd, scale)

    def timestral_rope_tables(self, groups, ne, l, h, hd, rope_dim, theta, first_obs):
        sl = ne + h
        c = np.empty(groups * sl * (hd // 2), np.float32)
        s = np.empty_like(c)
        fo = np.ascontiguousarray(first_obs, dtype=np.uintp)
        self.lib.orc_timestral_rope_tables(ptr(c), ptr(s), groups, ne, l, h, hd, rope_dim, theta, ptr(fo))
        return c, s

    def timestral_key_valid(self, obs, rows, vall, ne, ps, attend_missing=True):
        """(key_valid (rows, ne) uint8, first_obs (rows // vall) int, keys_all_valid bool)."""
        obs = np.ascontiguousarray(obs, np.uint8)
        assert obs.size == rows * ne * ps
        kv = np.zeros(rows * ne, np.uint8)
        fo = np.zeros(max(rows // vall, 1), np.uintp)
        all_valid = self.lib.orc_timestral_key_valid(ptr(kv), ptr(fo), ptr(obs), rows, vall, ne, ps,
                                                     int(attend_missing))
        return kv.reshape(rows, ne), fo[: rows // vall].astype(np.int64), bool(all_valid)

    def timestral_rope(self, threads, qkv, cos_t, sin_t, rows, sl, vall, d, nh, hd):
        self.lib.orc_timestral_rope(threads, ptr(qkv), ptr(cos_t), ptr(sin_t), rows, sl, vall, d, nh, hd)

    def timestral_time_attention(self, threads, qkv, o, key_valid, keys_all_valid, bidir, rows, ne, l, h, d, nh, hd):
        self.lib.orc_timestral_time_attention(threads, ptr(qkv), ptr(o), ptr(key_valid), int(keys_all_valid),
                                              ptr(bidir), rows, ne, l, h, d, nh, hd)

    def timestral_variate_attention(self, threads, qkv, o, key_valid, roles, cov, groups, vall, ne, h, d, nh, hd):
        self.lib.orc_timestral_variate_attention(threads, ptr(qkv), ptr(o), ptr(key_valid), ptr(roles), int(cov), groups,
                                                 vall, ne, h, d, nh, hd)

    def mul_sigmoid(self, dst, x, g):
        self.lib.orc_mul_sigmoid(ptr(dst), ptr(x), ptr(g), x.size)

    def batched_self_attend(self, threads, mask, q, q_tok, q_batch, k, k_tok, k_batch, v, v_tok, v_batch, o, o_tok,
                            o_batch, key_valid, kv_batch, bias, nb, nh, n, hd, scale):
        self.lib.orc_batched_self_attend(threads, mask, ptr(q), q_tok, q_batch, ptr(k), k_tok, k_batch, ptr(v), v_tok,
                                         v_batch, ptr(o), o_tok, o_batch, ptr(key_valid), kv_batch, ptr(bias), nb, nh,
                                         n, hd, scale)

    # ---- Timestral model and forecaster ----------------------------------------------------------

    def silu_in_place(self, x):
        self.lib.orc_silu_in_place(ptr(x), x.size)

    def mul_silu(self, dst, gate, up):
        self.lib.orc_mul_silu(ptr(dst), ptr(gate), ptr(up), dst.size)

    def softplus(self, x):
        return self.lib.orc_softplus(x)

    def clamp_nonfinite(self, v):
        self.lib.orc_clamp_nonfinite(ptr(v), v.size)

    def resblock_silu(self, threads, y, x, rows, rb):
        st = resblock_struct(rb)
        self.lib.orc_resblock_silu(threads, ptr(y), ptr(x), rows, ctypes.byref(st))

    def timestral_patch_stats(self, threads, data, obs, rows, t, ps, min_scale):
        data = np.ascontiguousarray(data, np.float32)
        obs = np.ascontiguousarray(obs, np.uint8)
        loc = np.zeros(rows * (t // ps), np.float32)
        scale = np.zeros_like(loc)
        self.lib.orc_timestral_patch_stats(threads, ptr(loc), ptr(scale), ptr(data), ptr(obs), rows, t, ps, min_scale)
        return loc.reshape(rows, -1), scale.reshape(rows, -1)

    def timestral_predict_block(self, threads, m, ctx, obs, t, groups, vall, h):
        ctx = np.ascontiguousarray(ctx, np.float32)
        obs = np.ascontiguousarray(obs, np.uint8)
        out = np.zeros((groups * vall, h * m["ps"], m["q"]), np.float32)
        st = timestral_model_struct(m)
        self.lib.orc_timestral_predict_block(threads, ptr(out), ctypes.byref(st), ptr(ctx), ptr(obs), t, groups, vall, h)
        return out

    def timestral_predict_block_cov(self, threads, m, ctx, obs, t, groups, vall, h, roles, kf=None, kfm=None):
        """(groups * targets, h * ps, q) quantiles of the target rows."""
        ctx = np.ascontiguousarray(ctx, np.float32)
        obs = np.ascontiguousarray(obs, np.uint8)
        roles = np.ascontiguousarray(roles, np.uint8)
        kf = None if kf is None else np.ascontiguousarray(kf, np.float32)
        kfm = None if kfm is None else np.ascontiguousarray(kfm, np.uint8)
        out = np.zeros((groups * int((roles == 0).sum()), h * m["ps"], m["q"]), np.float32)
        st = timestral_model_struct(m)
        self.lib.orc_timestral_predict_block_cov(threads, ptr(out), ctypes.byref(st), ptr(ctx), ptr(obs), t, groups,
                                                 vall, h, ptr(roles), None if kf is None else ptr(kf),
                                                 None if kfm is None else ptr(kfm))
        return out

    def timestral_forecast_cov(self, threads, m, inputs, observed, b, v, t, horizon, past=None, known=None,
                               max_context=0, per_shot=32, cap_k=1e4, extreme=1e30, symmetric=True,
                               clip_nonnegative=True):
        """(rc, out (b, v, horizon, q)); past (b, n_past, t), known (b, n_known, t + horizon), NaN = missing."""
        inputs = np.ascontiguousarray(inputs, np.float32)
        observed = np.ascontiguousarray(observed, np.uint8)
        past = None if past is None else np.ascontiguousarray(past, np.float32)
        known = None if known is None else np.ascontiguousarray(known, np.float32)
        n_past = 0 if past is None else past.shape[1]
        n_known = 0 if known is None else known.shape[1]
        out = np.zeros((b, v, horizon, m["q"]), np.float32)
        st = timestral_model_struct(m)
        rc = self.lib.orc_timestral_forecast_cov(threads, ptr(out), ctypes.byref(st), ptr(inputs), ptr(observed), b,
                                                 v, t, horizon, None if past is None else ptr(past), n_past,
                                                 None if known is None else ptr(known), n_known, max_context,
                                                 per_shot, cap_k, extreme, int(symmetric), int(clip_nonnegative))
        return rc, out

    def timestral_encode_categorical(self, codes, inputs, observed, max_context):
        """codes (b, c, len) f64, inputs / observed (b, v, t) -> (b, c, len) f32."""
        codes = np.ascontiguousarray(codes, np.float64)
        inputs = np.ascontiguousarray(inputs, np.float32)
        observed = np.ascontiguousarray(observed, np.uint8)
        b, c, n = codes.shape
        out = np.zeros((b, c, n), np.float32)
        self.lib.orc_timestral_encode_categorical(ptr(out), ptr(codes), b, c, n, ptr(inputs), ptr(observed),
                                                  inputs.shape[1], inputs.shape[2], max_context)
        return out

    def timestral_refine_block(self, qs, m, ctx, obs, rows, t, h):
        st = timestral_model_struct(m)
        ctx = np.ascontiguousarray(ctx, np.float32)  # held here: the call reads through raw pointers
        obs = np.ascontiguousarray(obs, np.uint8)
        self.lib.orc_timestral_refine_block(ptr(qs), ctypes.byref(st), ptr(ctx), ptr(obs), rows, t, h)

    def timestral_forecast(self, threads, m, inputs, observed, b, v, t, horizon, max_context=0, per_shot=32,
                           cap_k=1e4, extreme=1e30, symmetric=True, clip_nonnegative=True):
        """(rc, out (b, v, horizon, q))."""
        inputs = np.ascontiguousarray(inputs, np.float32)
        observed = np.ascontiguousarray(observed, np.uint8)
        out = np.zeros((b, v, horizon, m["q"]), np.float32)
        st = timestral_model_struct(m)
        rc = self.lib.orc_timestral_forecast(threads, ptr(out), ctypes.byref(st), ptr(inputs), ptr(observed), b, v, t,
                                             horizon, max_context, per_shot, cap_k, extreme, int(symmetric),
                                             int(clip_nonnegative))
        return rc, out

