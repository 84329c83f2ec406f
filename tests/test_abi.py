"""CPU-side checks of the C ABI (no GPU needed): exports, host functions, argument validation and
the "return non-zero so the caller uses the CPU" contract (src/platform/backend.zig:33-36)."""
import ctypes
import json
import os
import pathlib
import re
import subprocess
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tsfm_attn.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(tsfm_\w+)\s*\(", text)))


def test_header_and_binding_agree(ta):
    assert sorted(ta.EXPORTS) == declared_functions()


def test_library_exports_every_declared_symbol(ta):
    out = subprocess.run(["nm", "-D", "--defined-only", str(ta.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (tsfm_\w+)", out.stdout))
    missing = [f for f in declared_functions() if f not in exported]
    assert not missing, missing


@pytest.mark.parametrize("struct,cname", [("AttnArgs", "tsfm_attn_args"), ("VariateArgs", "tsfm_variate_args"),
                                          ("ProjArgs", "tsfm_proj_args"), ("Chronos2Layer", "tsfm_chronos2_layer"),
                                          ("Chronos2EncodeArgs", "tsfm_chronos2_encode_args"),
                                          ("Resblock", "tsfm_resblock"),
                                          ("Chronos2ForwardArgs", "tsfm_chronos2_forward_args"),
                                          ("BoltEncLayer", "tsfm_bolt_enc_layer"), ("BoltDecLayer", "tsfm_bolt_dec_layer"),
                                          ("BoltForwardArgs", "tsfm_bolt_forward_args"),
                                          ("BoltForecastArgs", "tsfm_bolt_forecast_args"),
                                          ("BoltHorizonArgs", "tsfm_bolt_horizon_args"),
                                          ("Chronos2ForecastArgs", "tsfm_chronos2_forecast_args"),
                                          ("TimestralAttn", "tsfm_timestral_attn"),
                                          ("TimestralLayer", "tsfm_timestral_layer"),
                                          ("TimestralModel", "tsfm_timestral_model"),
                                          ("TimestralForecastArgs", "tsfm_timestral_forecast_args")])
def test_args_struct_layout_matches_header(ta, struct, cname):
    """Compile a tiny C program against the header and compare offsetof() with the ctypes struct."""
    cls = getattr(ta, struct)
    fields = [f[0] for f in cls._fields_]
    src = "#include <stdio.h>\n#include <stddef.h>\n#include \"tsfm_attn.h\"\nint main(void){\n"
    src += f'printf("%zu\\n", sizeof({cname}));\n'
    for f in fields:
        src += f'printf("%zu\\n", offsetof({cname}, {f}));\n'
    src += "return 0;}\n"
    tmp = pathlib.Path(os.environ.get("TMPDIR", "/tmp")) / f"tsfm_layout_{os.getpid()}_{cname}"
    tmp.mkdir(exist_ok=True)
    (tmp / "l.c").write_text(src)
    subprocess.run(["gcc", "-I", str(ROOT / "include"), "-o", str(tmp / "l"), str(tmp / "l.c")], check=True)
    got = [int(x) for x in subprocess.run([str(tmp / "l")], capture_output=True, text=True, check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(cls)
    assert got[1:] == [getattr(cls, f).offset for f in fields]


def test_t5_bucket_host_function_golden(ta):
    g = json.loads((ROOT / "tests" / "golden" / "t5_buckets_32_128.json").read_text())
    lib = ta.load()
    got = [lib.tsfm_t5_relative_bucket(g["rel_first"] + i, 32, 128) for i in range(len(g["buckets"]))]
    assert got == g["buckets"]
    # The table form used by the kernel: out[t] = bucket(t - (n_q - 1)).
    n_q, n_k = 129, 129
    out = np.zeros(n_q + n_k - 1, np.int32)
    assert lib.tsfm_t5_bucket_table(out.ctypes.data, n_q, n_k, 32, 128) == ta.OK
    rel = np.arange(-(n_q - 1), n_k)
    sel = (rel >= -140) & (rel <= 140)
    assert out[sel].tolist() == [g["buckets"][r + 140] for r in rel[sel]]


def test_mask_pick_mirror():
    sys.path.insert(0, str(ROOT / "tsfm-zig_amd"))
    import tsfm_attn

    g = json.loads((ROOT / "tests" / "golden" / "mask_pick.json").read_text())
    for c in g["cases"]:
        assert tsfm_attn.Mask.pick(c["causal"], c["all_keys_valid"], c["additive"]).name.lower() == c["mask"]


def _valid_host_args(ta, **over):
    n, H = 8, 2
    bufs = {name: np.zeros(n * H * 64, np.float32) for name in "qkvo"}
    kw = dict(q=bufs["q"], k=bufs["k"], v=bufs["v"], o=bufs["o"], mask=ta.Mask.FULL, batch=1, heads=H, n_q=n,
              n_k=n, q_tok=H * 64, q_batch=0, k_tok=H * 64, k_batch=0, v_tok=H * 64, v_batch=0, o_tok=H * 64,
              o_batch=0, scale=0.125)
    kw.update(over)
    return ta.make_args(**kw), bufs


@pytest.mark.parametrize("over,code", [
    (dict(head_dim=32), 2),
    (dict(mask=7), 3),
    (dict(q_tok=130), 2),
    (dict(mask=1), 3),            # keys_additive without key_valid
    (dict(q_pos0=-1), 3),
    (dict(dtype=2, scale=-0.5), 2),  # half precision takes the row max before scaling
    (dict(k_tok=1 << 26), 2),        # K rows of one series past 32-bit byte offsets
])
def test_validation_codes(ta, over, code):
    args, _ = _valid_host_args(ta, **over)
    assert ta.fwd(args) == code
    assert ta.last_error()


def test_empty_batch_is_a_no_op(ta):
    args, _ = _valid_host_args(ta, batch=0)
    assert ta.fwd(args) == ta.OK


def test_disabled_library_reports_unavailable():
    """With TSFM_HIP_DISABLE set every call returns E_UNAVAILABLE (the CPU-fallback signal), in a
    fresh process so the one-time initialisation sees the variable."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import numpy as np, tsfm_attn as ta\n"
        "assert ta.available() is False\n"
        "b = {c: np.zeros(8*64, np.float32) for c in 'qkvo'}\n"
        "a = ta.make_args(q=b['q'], k=b['k'], v=b['v'], o=b['o'], mask=0, batch=1, heads=1, n_q=8, n_k=8,"
        " q_tok=64, q_batch=0, k_tok=64, k_batch=0, v_tok=64, v_batch=0, o_tok=64, o_batch=0, scale=1.0)\n"
        "rc = ta.fwd(a)\n"
        "assert rc == ta.E_UNAVAILABLE, rc\n"
        "assert 'TSFM_HIP_DISABLE' in ta.last_error()\n"
    ) % str(ROOT / "tsfm-zig_amd")
    env = dict(os.environ, TSFM_HIP_DISABLE="1")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_kv_cache_rejects_f32(ta):
    lib = ta.load()
    h = ctypes.c_void_p()
    assert lib.tsfm_kv_create(ctypes.byref(h), ta.DTYPE_F32, 1, 1, 64, 32) == ta.E_UNSUPPORTED
    assert not h.value


def _variate_host_args(ta, **over):
    groups, vall, ne, h, nh = 2, 3, 5, 2, 2
    sl, d = ne + h, nh * 64
    qkv = np.zeros(groups * vall * sl * 3 * d, np.float32)
    o = np.zeros(groups * vall * sl * d, np.float32)
    kv = np.ones(groups * vall * ne, np.uint8)
    kw = dict(dtype=ta.DTYPE_F32, groups=groups, vall=vall, n_tok=sl, n_enc=ne, heads=nh, head_dim=64, cov=1,
              scale=0.125, qkv=qkv.ctypes.data, qkv_row=sl * 3 * d, qkv_tok=3 * d, o=o.ctypes.data, o_row=sl * d,
              o_tok=d, key_valid=kv.ctypes.data, kv_row=ne)
    kw.update(over)
    roles = kw.pop("roles", [0, 1, 2])
    a = ta.VariateArgs(**kw)
    role_bytes = None
    if roles is not None:
        role_bytes = (ctypes.c_uint8 * max(len(roles), kw["vall"], 1))(*roles)
        a.roles = role_bytes
    return a, (qkv, o, kv, role_bytes)


@pytest.mark.parametrize("over,code", [
    (dict(vall=257), 2),           # more rows than the kernels' role words hold
    (dict(roles=None), 3),         # roles are required with cov
    (dict(dtype=2), 2),            # f32 only
    (dict(head_dim=32), 2),
    (dict(n_enc=9), 3),            # more encoder slots than tokens
    (dict(roles=[0, 3, 1]), 3),    # not a model.Role
    (dict(key_valid=None), 3),
    (dict(o_tok=130), 2),          # strides in whole 16-byte units
])
def test_variate_validation_codes(ta, over, code):
    a, _keep = _variate_host_args(ta, **over)
    assert ta.variate_attend(a) == code
    assert ta.last_error()


def test_variate_empty_is_a_no_op(ta):
    a, _keep = _variate_host_args(ta, groups=0)
    assert ta.variate_attend(a) == ta.OK


def _proj_host_args(ta, **over):
    b, seq, d_in, nh = 2, 5, 64, 2
    width = nh * 64
    x = np.zeros(b * seq * d_in, np.float32)
    w = np.zeros(width * d_in, np.float32)
    y = np.zeros(b * seq * width, np.float32)
    tab = np.zeros(seq * 32, np.float32)
    kw = dict(dtype=ta.DTYPE_F32, batch=b, seq=seq, d_in=d_in, heads=nh, head_dim=64, rope_half=32,
              x=x.ctypes.data, x_tok=d_in, w_q=w.ctypes.data, w_k=w.ctypes.data, w_v=w.ctypes.data,
              q=y.ctypes.data, q_tok=width, k=y.ctypes.data, k_tok=width, v=y.ctypes.data, v_tok=width,
              rope_cos=tab.ctypes.data, rope_sin=tab.ctypes.data)
    kw.update(over)
    return ta.ProjArgs(**kw), (x, w, y, tab)


@pytest.mark.parametrize("over,code", [
    (dict(dtype=1), 2),                 # f32 only
    (dict(head_dim=32), 2),
    (dict(d_in=40, x_tok=40), 2),       # d_in not a multiple of 16
    (dict(x_tok=66), 2),                # stride not a multiple of 16 bytes
    (dict(batch=-1), 3),
    (dict(w_k=None), 3),
    (dict(rope_sin=None), 3),           # rope_cos without rope_sin
    (dict(rope_half=16), 3),            # tables must be head_dim / 2 wide
    (dict(x_tok=32), 3),                # token stride shorter than d_in
    (dict(q_tok=64), 3),                # token stride shorter than heads * 64
    (dict(w_gate=1 << 20), 3),          # w_gate without gate
    (dict(out_dtype=3), 3),             # not a TSFM_DTYPE_*
])
def test_proj_validation_codes(ta, over, code):
    a, _keep = _proj_host_args(ta, **over)
    assert ta.qkv_project(a) == code
    assert ta.last_error()


def test_proj_empty_is_a_no_op(ta):
    for over in (dict(batch=0), dict(seq=0), dict(heads=0)):
        a, _keep = _proj_host_args(ta, **over)
        assert ta.qkv_project(a) == ta.OK


@pytest.mark.parametrize("m,n,k,lda,ldb,ldc,code", [
    (0, 8, 16, 16, 16, 8, 3),     # empty: the caller's CPU path (cuda_sgemm_nt returns -1 too)
    (4, 8, 16, 12, 16, 8, 3),     # lda < k
    (4, 8, 24, 24, 24, 8, 2),     # k not a multiple of 16
    (4, 6, 16, 16, 16, 8, 2),     # n not a multiple of 4
    (4, 8, 16, 18, 16, 8, 2),     # lda not a multiple of 4
])
def test_sgemm_nt_argument_codes(ta, m, n, k, lda, ldb, ldc, code):
    a = np.zeros(max(m, 1) * lda, np.float32)
    b = np.zeros(n * ldb, np.float32)
    c = np.zeros(max(m, 1) * ldc, np.float32)
    assert ta.sgemm_nt(m, n, k, 1.0, a, lda, b, ldb, c, ldc) == code
    assert ta.last_error()


@pytest.mark.parametrize("m,n,k,lda,ldb,ldc,code", [
    (0, 4, 16, 16, 4, 4, 3),      # empty product
    (4, 4, 16, 8, 4, 4, 3),       # lda < k
    (4, 8, 16, 16, 4, 8, 3),      # ldb < n
    (4, 8, 16, 16, 8, 4, 3),      # ldc < n
    (4, 4, 12, 12, 4, 4, 2),      # k not a multiple of 16
    (4, 6, 16, 16, 6, 6, 2),      # n not a multiple of 4
    (4, 4, 16, 18, 4, 4, 2),      # lda not a multiple of 4
])
def test_sgemm_nn_argument_codes(ta, m, n, k, lda, ldb, ldc, code):
    """cuda_sgemm_nn's arguments (src/platform/cuda/gemm.c:324-330): B is [k][ldb]."""
    a = np.zeros(max(m, 1) * lda, np.float32)
    b = np.zeros(k * ldb, np.float32)
    c = np.zeros(max(m, 1) * ldc, np.float32)
    assert ta.sgemm_nn(m, n, k, a, lda, b, ldb, c, ldc) == code
    assert ta.last_error()


def _encode_args(ta, **over):
    d, seq, b = 128, 4, 2
    x = np.zeros(b * seq * d, np.float32)
    kv = np.ones(b * seq, np.uint8)
    tab = np.zeros(seq * 32, np.float32)
    w = np.zeros(512 * 128, np.float32)
    arr = (ta.Chronos2Layer * 1)()
    for f in ta.CHRONOS2_LAYER_FIELDS:
        setattr(arr[0], f, w.ctypes.data)
    kw = dict(batch=b, seq=seq, d_model=d, heads=2, head_dim=64, d_ff=256, n_layers=1, keys_all_valid=1, eps=1e-6,
              scale=1.0, x=x.ctypes.data, key_valid=kv.ctypes.data, rope_cos=tab.ctypes.data,
              rope_sin=tab.ctypes.data, layers=arr, final_norm=w.ctypes.data)
    kw.update(over)
    return ta.Chronos2EncodeArgs(**kw), (x, kv, tab, w, arr)


@pytest.mark.parametrize("over,code", [
    (dict(head_dim=32, d_model=64), 2),
    (dict(d_model=130), 3),          # not heads * head_dim
    (dict(d_ff=100), 2),             # not a multiple of 16
    (dict(x=None), 3),
    (dict(key_valid=None), 3),
    (dict(layers=None), 3),
    (dict(batch=-1), 3),
])
def test_encode_validation_codes(ta, over, code):
    a, _keep = _encode_args(ta, **over)
    assert ta.load().tsfm_chronos2_encode(ctypes.byref(a)) == code
    assert ta.last_error()


def test_encode_null_layer_weight_is_invalid(ta):
    a, keep = _encode_args(ta)
    keep[4][0].mlp_wo = None
    assert ta.load().tsfm_chronos2_encode(ctypes.byref(a)) == ta.E_INVALID


def test_encode_empty_is_a_no_op(ta):
    a, _keep = _encode_args(ta, batch=0)
    assert ta.load().tsfm_chronos2_encode(ctypes.byref(a)) == ta.OK


def test_bolt_forecast_is_device_only(ta):
    """The forecast's preparation and inverse norm run on the device: host pointers are refused
    (before any device work), and a NULL argument block is invalid."""
    lib = ta.load()
    assert lib.tsfm_bolt_forecast(None) == ta.E_INVALID
    ctx = np.zeros(64, np.float32)
    out = np.zeros(64, np.float32)
    a = ta.BoltForecastArgs(ctx=ctx.ctypes.data, stride=64, len=64, patch=16, norm_eps=1e-5, out=out.ctypes.data)
    a.model.batch = 1
    a.model.n_patch = 4
    assert lib.tsfm_bolt_forecast(ctypes.byref(a)) == ta.E_UNSUPPORTED
    assert "device" in ta.last_error()


def test_chronos2_forecast_is_device_only(ta):
    lib = ta.load()
    assert lib.tsfm_chronos2_forecast(None) == ta.E_INVALID
    x = np.zeros(64, np.float32)
    a = ta.Chronos2ForecastArgs(inputs=x.ctypes.data, stride=64, len=64, horizon=16, time_scale=1.0,
                                out=x.ctypes.data)
    a.model.enc.batch = 1
    assert lib.tsfm_chronos2_forecast(ctypes.byref(a)) == ta.E_UNSUPPORTED
    assert "device" in ta.last_error()


def _timestral_args(ta, **over):
    """A tsfm_timestral_forecast_args block that passes validation up to the device: host buffers
    stand in for the device pointers (validation reads only the host-side knots and layers)."""
    buf = np.zeros(4096, np.float32)
    knots = np.array([0.1, 0.5, 0.9])
    layers = (ta.TimestralLayer * 1)()
    layers[0].n_attn = 1
    layers[0].attn[0] = ta.TimestralAttn(1, buf.ctypes.data, buf.ctypes.data, buf.ctypes.data, None)
    layers[0].mlp_norm = layers[0].w12 = layers[0].w3 = buf.ctypes.data
    def rb(i, h, o, biases):
        r = ta.Resblock(**{f: buf.ctypes.data for f in ta.RESBLOCK_FIELDS})
        if not biases:
            r.hidden_b = r.output_b = r.residual_b = None
        r.__setattr__("in", i)
        r.hid, r.out, r.act = h, o, 1
        return r
    m = ta.TimestralModel(patch=16, d_model=128, heads=2, head_dim=64, mlp_hidden=256, n_layers=1, n_quantiles=3,
                          block_size=32, context_length=2048, rope_dim=32, use_asinh=1, attend_missing=1,
                          covariate_enabled=1, rope_theta=1e4, norm_eps=1e-6, minimum_scale=1e-6,
                          quantile_width_factor=2.0, quantile_knots=knots.ctypes.data, patch_proj=rb(32, 512, 128, True),
                          head=rb(128, 512, 48, False), forecast_query=buf.ctypes.data, out_norm=buf.ctypes.data,
                          layers=layers)
    a = ta.TimestralForecastArgs(model=m, inputs=buf.ctypes.data, observed=buf.ctypes.data, batch=1, variates=1,
                                 len=64, horizon=16, quantile_real_cap_k=1e4, extreme_value_threshold=1e30,
                                 symmetric_averaging=1, clip_nonnegative=1, kv_cache=1, flags=ta.DEVICE_PTRS,
                                 out=buf.ctypes.data)
    for k, v in over.items():
        setattr(a, k, v)
    return a, (buf, knots, layers)


def test_timestral_forecast_validation_matches_the_reference_errors(ta):
    """forecaster.zig:83-104 and the build's own limits, decided before any device work: a
    covariate array with no rows is error.InvalidInput (TSFM_E_INVALID), covariates on a model with
    covariate_enabled off are error.CovariatesUnsupported, row counts near INT32_MAX are refused
    without overflow, and bf16 time attention with use_asinh is refused."""
    lib = ta.load()
    f = lambda a: lib.tsfm_timestral_forecast(ctypes.byref(a))
    buf = np.zeros(64, np.float32)
    a, keep = _timestral_args(ta, past=buf.ctypes.data, n_past=0)
    assert f(a) == ta.E_INVALID and "InvalidInput" in ta.last_error()
    a, keep = _timestral_args(ta, known=buf.ctypes.data, n_known=0)
    assert f(a) == ta.E_INVALID
    a, keep = _timestral_args(ta, n_known=2)  # a count without its array
    assert f(a) == ta.E_INVALID
    a, keep = _timestral_args(ta, past=buf.ctypes.data, n_past=(1 << 31) - 1)
    assert f(a) == ta.E_UNSUPPORTED  # 1 + INT32_MAX rows: refused, not wrapped
    a, keep = _timestral_args(ta, past=buf.ctypes.data, n_past=(1 << 31) - 1, known=buf.ctypes.data,
                              n_known=(1 << 31) - 1, variates=(1 << 31) - 1)
    assert f(a) == ta.E_UNSUPPORTED
    a, keep = _timestral_args(ta, past=buf.ctypes.data, n_past=1)
    a.model.covariate_enabled = 0
    assert f(a) == ta.E_UNSUPPORTED and "CovariatesUnsupported" in ta.last_error()
    a, keep = _timestral_args(ta, flags=ta.DEVICE_PTRS | ta.TIMESTRAL_BF16_ATTN)
    assert f(a) == ta.E_UNSUPPORTED and "use_asinh" in ta.last_error()
    if not ta.available():  # host buffers stand in for device memory: never launched
        a, keep = _timestral_args(ta)
        assert f(a) == ta.E_UNAVAILABLE  # the unchanged block passes validation, stops at the device


_FUZZ = r'''
import ctypes, math, os, random, sys
sys.path.insert(0, %r)
import numpy as np, tsfm_attn as ta
lib = ta.load(os.environ["TSFM_FUZZ_LIB"]) if os.environ.get("TSFM_FUZZ_LIB") else ta.load()
assert not lib.tsfm_attn_available()
rng = random.Random(20261202)
buf = np.zeros(1 << 16, np.float32)
kvb = np.ones(4096, np.uint8)
ints = [-(1 << 31), -5, -1, 0, 1, 2, 17, 64, 129, 577, 2048, (1 << 31) - 1]
strides = [-(1 << 63), -(1 << 40), -1, 0, 1, 64, 130, 768, 3072, 1 << 26, 1 << 40, (1 << 62)]
floats = [0.0, 0.125, 1.0, -0.5, math.inf, -math.inf, math.nan]
ptrs = [None, buf.ctypes.data]
codes = set()
def valid():
    row = 2 * 64
    return ta.make_args(q=buf, k=buf, v=buf, o=buf, mask=0, batch=2, heads=2, n_q=17, n_k=17, q_tok=row,
                        q_batch=17 * row, k_tok=row, k_batch=17 * row, v_tok=row, v_batch=17 * row, o_tok=row,
                        o_batch=17 * row, scale=0.125)
for it in range(2000):  # a valid block with one to three fields changed
    a = valid()
    for _ in range(rng.randint(1, 3)):
        f = rng.choice([n for n, _ in ta.AttnArgs._fields_ if n != "stream"])
        t = dict(ta.AttnArgs._fields_)[f]
        if t is ctypes.c_void_p:
            setattr(a, f, rng.choice(ptrs + [kvb.ctypes.data]))
        elif t is ctypes.c_float:
            setattr(a, f, rng.choice(floats))
        elif t is ctypes.c_int64:
            setattr(a, f, rng.choice(strides))
        elif t is ctypes.c_uint32:
            setattr(a, f, rng.choice([0, 2, 0xFFFFFFFE]))
        else:
            setattr(a, f, rng.choice(ints + [-1, 3, 5, 7, 99]))
    rc = lib.tsfm_attn_fwd(ctypes.byref(a))
    assert rc in (0, 1, 2, 3), (it, rc)
    codes.add(rc)
for it in range(2000):  # every field random
    a = ta.AttnArgs()
    a.dtype = rng.choice([-1, 0, 1, 2, 3, 99])
    a.mask = rng.choice(range(-1, 8))
    for f in ("batch", "heads", "n_q", "n_k", "q_pos0", "ctx_keys", "chain_start", "rel_buckets", "rope_half",
              "rope_rows_per_table", "rope_row0"):
        setattr(a, f, rng.choice(ints))
    a.head_dim = rng.choice([0, 16, 32, 64, 128, -64])
    a.scale = rng.choice(floats)
    a.flags = rng.choice([0, 2, 0xFFFFFFFE])
    for f in ("q_tok", "q_batch", "k_tok", "k_batch", "v_tok", "v_batch", "o_tok", "o_batch", "kv_batch",
              "bias_head", "bias_row", "rope_table_stride"):
        setattr(a, f, rng.choice(strides))
    for f in ("q", "k", "v", "o", "bias", "rel_table", "rel_bucket", "rope_cos", "rope_sin"):
        setattr(a, f, rng.choice(ptrs))
    a.key_valid = rng.choice([None, kvb.ctypes.data])
    rc = lib.tsfm_attn_fwd(ctypes.byref(a))
    assert rc in (0, 1, 2, 3), (it, rc)
    codes.add(rc)
def fill(a):
    for f, t in type(a)._fields_:
        if f == "stream" or not hasattr(t, "__mro__") or issubclass(t, ctypes.Array):
            continue
        if t is ctypes.c_void_p:
            setattr(a, f, rng.choice(ptrs))
        elif t is ctypes.c_float:
            setattr(a, f, rng.choice(floats))
        elif t is ctypes.c_int64:
            setattr(a, f, rng.choice(strides + [64, 128, 768, 3 * 768]))
        elif t is ctypes.c_uint32:
            setattr(a, f, rng.choice([0, 2, 0xFFFFFFFE]))
        elif t in (ctypes.c_int32, ctypes.c_int):
            setattr(a, f, rng.choice(ints + [0, 1, 2, 3, 4, 16, 64, 64, 64]))
for cls, fn in ((ta.VariateArgs, lib.tsfm_variate_attend), (ta.ProjArgs, lib.tsfm_qkv_project)):
    fn.argtypes = [ctypes.POINTER(cls)]
    fn.restype = ctypes.c_int
    for it in range(3000):
        a = cls()
        fill(a)
        rc = fn(ctypes.byref(a))
        assert rc in (0, 1, 2, 3), (cls.__name__, it, rc)
        codes.add(rc)
fn = lib.tsfm_timestral_forecast
fn.argtypes = [ctypes.POINTER(ta.TimestralForecastArgs)]
fn.restype = ctypes.c_int
for it in range(3000):  # model and forecast fields random (counts near INT32_MAX included); no layers array
    a = ta.TimestralForecastArgs()
    fill(a)
    fill(a.model)
    rc = fn(ctypes.byref(a))
    assert rc in (0, 1, 2, 3), ("timestral", it, rc)
    codes.add(rc)
print(sorted(codes))
'''


def test_validation_fuzz_returns_codes_and_never_launches():
    """4000 random argument blocks (extreme dims and strides, null and short buffers, bad dtypes,
    masks, flags and scales) through tsfm_attn_fwd, and 3000 each through tsfm_variate_attend,
    tsfm_qkv_project and tsfm_timestral_forecast, in a fresh process with TSFM_HIP_DISABLE=1:
    every call returns one of the ABI's codes, and whatever passes validation stops at the
    disabled device instead of launching. Under the sanitizer run this is the check that the
    validation arithmetic has no overflow or out-of-bounds read."""
    env = dict(os.environ, TSFM_HIP_DISABLE="1")
    if os.environ.get("TSFM_TEST_PRODUCT_LIB"):
        env["TSFM_FUZZ_LIB"] = os.environ["TSFM_TEST_PRODUCT_LIB"]
    r = subprocess.run([sys.executable, "-c", _FUZZ % str(ROOT / "tsfm-zig_amd")], env=env, capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    seen = eval(r.stdout.strip().splitlines()[-1])
    assert {1, 2, 3} <= set(seen), seen  # unavailable (passed validation), unsupported, invalid all reached


def test_categorical_encoding_matches_the_oracle(ta, orc):
    """tsfm_timestral_encode_categorical (host) against the oracle's restatement, bit for bit: one
    and two target variates, past and known code lengths, windows, NaN / infinite / unseen codes,
    and the rows written at row0 of a wider per-series block (the numeric rows untouched)."""
    rng = np.random.default_rng(5)
    for trial in range(30):
        b, c, t = int(rng.integers(1, 4)), int(rng.integers(1, 4)), int(rng.integers(1, 90))
        h = int(rng.integers(0, 40)) if trial % 2 else 0
        v = 1 if trial % 3 else 2
        x = (rng.standard_normal((b, v, t)) * 5).astype(np.float32)
        ob = (rng.random((b, v, t)) < 0.7).astype(np.uint8)
        codes = rng.integers(0, 7, (b, c, t + h)).astype(np.float64) * 1.5
        codes[rng.random(codes.shape) < 0.2] = np.nan
        codes[rng.random(codes.shape) < 0.03] = -np.inf
        window = int(rng.integers(1, 120))
        want = orc.timestral_encode_categorical(codes, x, ob, window)
        got = ta.timestral_encode_categorical(codes, x, ob, window)
        assert np.array_equal(got, want, equal_nan=True), trial
        wide = np.full((b, c + 3, t + h), 7.0, np.float32)
        ta.timestral_encode_categorical(codes, x, ob, window, out=wide, row0=2)
        assert np.array_equal(wide[:, 2:2 + c], want, equal_nan=True)
        assert (wide[:, :2] == 7).all() and (wide[:, 2 + c:] == 7).all()


@pytest.mark.parametrize("over,msg", [
    (dict(max_context=0), "max_context"),
    (dict(row0=2), "outside"),             # rows 2..3 of 2
    (dict(len=3), "sizes"),                # shorter than t
    (dict(inputs=None), "inputs and observed"),
    (dict(codes=None), "out and codes"),
])
def test_categorical_encoding_errors(ta, over, msg):
    x = np.zeros((1, 1, 5), np.float32)
    ob = np.ones((1, 1, 5), np.uint8)
    codes = np.zeros((1, 2, 5))
    out = np.zeros((1, 2, 5), np.float32)
    kw = dict(out=out.ctypes.data, out_rows=2, row0=0, codes=codes.ctypes.data, batch=1, n_cat=2, len=5,
              inputs=x.ctypes.data, observed=ob.ctypes.data, variates=1, t=5, max_context=16)
    kw.update(over)
    a = ta.CategoricalArgs(**kw)
    assert ta.load().tsfm_timestral_encode_categorical(ta.ctypes.byref(a)) == ta.E_INVALID
    assert msg in ta.last_error()
