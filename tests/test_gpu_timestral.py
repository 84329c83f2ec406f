"""GPU parity of the Timestral forecaster (tsfm_timestral_forecast: forecastRaw, blockDecode with
predictBlock and refineBlock, the cap, the mirrored average and the clip on the device) against the
oracle's restatement of forecaster.forecast (src/timestral/forecaster.zig:57-180), which re-encodes
the whole grown context every decode block as the reference does, through the C ABI.

The device path runs with and without its KV cache (decode blocks after the first run only their
new patches and decoder tokens over the kept time-attention K/V). Bar: _ref.reference_bar against
the oracle's 16-lane build: twice the reference's own spread between its 8-lane and 16-lane builds
on the same forecast (at least 1e-5). Covered: one refined block, several blocks with median
feedback, a max_context window that drops its oldest steps, a series with no observation (cached
and uncached decoding agree), missing values and leading gaps, several variates per series,
numeric covariates in f32 and with the bf16 time attention.
"""
import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu

THREADS = 16


def _device_model(m):
    import torch

    def cu(x):
        return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()

    dm = dict(m)
    dm["patch_proj"] = {k: cu(v) for k, v in m["patch_proj"].items()}
    dm["head"] = {k: cu(v) for k, v in m["head"].items()}
    dm["forecast_query"], dm["out_norm"] = cu(m["forecast_query"]), cu(m["out_norm"])
    dm["layers"] = [dict(attns=[{k: (cu(v) if isinstance(v, np.ndarray) else v) for k, v in a.items()}
                                for a in ly["attns"]],
                         mlp_norm=cu(ly["mlp_norm"]), w12=cu(ly["w12"]), w3=cu(ly["w3"])) for ly in m["layers"]]
    return dm


def _case(seed, b=3, v=2, length=150, nan_frac=0.1, schedule=("time_variate", "time")):
    rng = np.random.default_rng(seed)
    m = _ref.timestral_model(rng, d=128, nh=2, hid=256, schedule=schedule)
    t = np.arange(length)
    x = (20 + 6 * np.sin(2 * np.pi * t / 24) + 0.02 * t + rng.standard_normal((b * v, length))).astype(np.float32)
    obs = rng.random((b * v, length)) >= nan_frac
    obs[:v, :37] = False  # the first series starts late
    x[~obs] = 0
    return m, x, obs


def _gpu(ta, m, x, obs, b, v, horizon, **kw):
    import torch

    out = torch.full((b, v, horizon, m["q"]), -7.0, device="cuda")
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    od = torch.from_numpy(np.ascontiguousarray(obs.astype(np.uint8))).cuda()
    rc = ta.timestral_forecast(out, xd, od, _device_model(m), b, v, x.shape[1], horizon, **kw)
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _oracle(orc, m, x, obs, b, v, horizon, max_context=0, per_shot=32):
    rc, out = orc.timestral_forecast(THREADS, m, x, obs, b, v, x.shape[1], horizon, max_context, per_shot)
    assert rc == 0
    return out


@pytest.mark.parametrize("kv_cache", [True, False])
@pytest.mark.parametrize("horizon,per_shot,max_context", [(40, 32, 0), (100, 2, 0), (100, 2, 176)])
def test_timestral_forecast_matches_reencoding_oracle(ta, orc, orc16, gpu_ready, kv_cache, horizon, per_shot,
                                                      max_context):
    b, v = 3, 2
    m, x, obs = _case(horizon + per_shot)
    got = _gpu(ta, m, x, obs, b, v, horizon, max_context=max_context, per_shot=per_shot, kv_cache=kv_cache)
    w8, w16 = (_oracle(o_, m, x, obs, b, v, horizon, max_context, per_shot) for o_ in (orc, orc16))
    exact = _ref.timestral_forecast_f64(m, x, obs, b, v, horizon, per_shot=per_shot, max_context=max_context)
    assert np.isfinite(got).all()
    _ref.assert_within_reference_bar(got, w8, w16, exact)


def test_timestral_cached_decode_equals_reencoding(ta, gpu_ready):
    """Several decode blocks: the cached path (only new patches and decoder tokens per block) and
    the re-encoding path give the same forecasts up to f32 summation order."""
    b, v, horizon = 2, 3, 160
    m, x, obs = _case(21, b, v)
    cached = _gpu(ta, m, x, obs, b, v, horizon, per_shot=4, kv_cache=True)
    full = _gpu(ta, m, x, obs, b, v, horizon, per_shot=4, kv_cache=False)
    assert _ref.scaled_err(cached, full) < 2e-5


@pytest.mark.parametrize("kv_cache", [True, False])
def test_timestral_bf16_time_attention(ta, orc16, gpu_ready, kv_cache):
    """TSFM_TIMESTRAL_BF16_ATTN: the time attention on the bf16 matrix cores over a bf16 K/V cache
    (q/k/v rounded once after RoPE, f32 softmax and accumulation, the output rounded once),
    everything else f32. Against the 16-lane oracle's f32 re-encoding forecast, scaled by
    max(|forecast|, 1): within 1e-2, the half-precision bar (measured about 5e-4). The model has
    use_asinh off: with it on, the head's outputs are sinh-expanded, so a random-init head's large
    outputs turn bf16's 2^-9 relative rounding into a few per cent of the forecast (measured
    2.5e-2 to 5e-2 for these weights) -- the bf16 rounding itself, not the decode. Cached and
    re-encoded bf16 decoding give the same forecast."""
    _, x, obs = _case(15, b=2, v=2)
    m = _ref.timestral_model(np.random.default_rng(5), d=128, nh=2, hid=256, use_asinh=False)
    b, v, horizon = 2, 2, 40
    want = _oracle(orc16, m, x, obs, b, v, horizon, per_shot=4)
    got = _gpu(ta, m, x, obs, b, v, horizon, per_shot=4, kv_cache=kv_cache, attn_bf16=True)
    assert np.isfinite(got).all()
    err = _ref.scaled_err(got, want)
    assert err < 1e-2, err
    f32 = _gpu(ta, m, x, obs, b, v, horizon, per_shot=4, kv_cache=kv_cache)
    assert _ref.scaled_err(f32, want) < err  # the bf16 rounding is what moves the forecast
    if kv_cache:
        full = _gpu(ta, m, x, obs, b, v, horizon, per_shot=4, kv_cache=False, attn_bf16=True)
        assert _ref.scaled_err(got, full) < 2e-5


@pytest.mark.parametrize("v", [1, 2])
def test_timestral_series_without_observation(ta, orc, orc16, gpu_ready, v):
    """A series with no observation at all: its RoPE origin (the first observed patch) moves once
    the medians are fed back. Its earlier tokens are invalid keys for every later query, so the
    cached decode (RoPE tables recomputed per block, no host round trip) stays the re-encoding's
    computation: it matches the oracle, and the uncached decode."""
    b, horizon = 2, 64
    m, x, obs = _case(5, b, v)
    obs[v:2 * v] = False
    x[v:2 * v] = 0
    got = _gpu(ta, m, x, obs, b, v, horizon, per_shot=2, kv_cache=True)
    full = _gpu(ta, m, x, obs, b, v, horizon, per_shot=2, kv_cache=False)
    w8, w16 = (_oracle(o_, m, x, obs, b, v, horizon, 0, 2) for o_ in (orc, orc16))
    exact = _ref.timestral_forecast_f64(m, x, obs, b, v, horizon, per_shot=2)
    _ref.assert_within_reference_bar(got, w8, w16, exact)
    assert _ref.scaled_err(got, full) < 2e-5
    assert _ref.scaled_err(got[1], w16[1]) < 1e-8  # the series without observation: the same bits as re-encoding


def test_timestral_forecast_accuracy_class(ta, orc, orc16, gpu_ready):
    """How far the device forecast is from a float64 evaluation (_ref.timestral_forecast_f64, the
    forecast composed from float64 definitions), against the reference's own two builds, over eight
    inputs (seeds 5-8, one and two variates, a series without observation, several decode blocks),
    cached and re-encoded.
    - In linear space (use_asinh off) every case is within the 1e-5 parity target of the 16-lane
      oracle (measured at most 1.4e-6).
    - In asinh space the head's outputs are sinh-expanded, so the forecast's scaled error is the
      absolute f32 error of the head's output: every f32 evaluation, the reference's included, is
      about 1e-6 to 7e-5 from float64 here, and two of them can differ by twice that on one input.
      Over the eight inputs, the device's largest distance from float64 is at most the reference's
      largest (measured 7.05e-5 against 7.23e-5): the same accuracy class, not a looser one."""
    b, horizon = 2, 64
    worst = {"gpu": 0.0, "ref": 0.0}
    for asinh in (False, True):
        for v in (1, 2):
            for seed in (5, 6, 7, 8):
                m, x, obs = _case(seed, b, v)
                if not asinh:
                    m = _ref.timestral_model(np.random.default_rng(seed), d=128, nh=2, hid=256, use_asinh=False)
                obs[v:2 * v] = False
                x[v:2 * v] = 0
                exact = _ref.timestral_forecast_f64(m, x, obs, b, v, horizon, per_shot=2)
                w8, w16 = (_oracle(o_, m, x, obs, b, v, horizon, 0, 2) for o_ in (orc, orc16))
                for kv_cache in (True, False):
                    got = _gpu(ta, m, x, obs, b, v, horizon, per_shot=2, kv_cache=kv_cache)
                    if not asinh:
                        assert _ref.scaled_err(got, w16) <= 1e-5, (v, seed, kv_cache)
                    else:
                        worst["gpu"] = max(worst["gpu"], _ref.scaled_err(got, exact))
                if asinh:
                    worst["ref"] = max(worst["ref"], _ref.scaled_err(w8, exact), _ref.scaled_err(w16, exact))
    print(f"asinh space, largest distance from float64: device {worst['gpu']:.3e}, reference {worst['ref']:.3e}")
    assert worst["gpu"] <= worst["ref"]


def test_timestral_forecast_argument_errors(ta, gpu_ready):
    import torch

    b, v, horizon = 1, 1, 16
    m, x, obs = _case(3, b, v)
    out = torch.zeros((b, v, horizon, m["q"]), device="cuda")
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    od = torch.from_numpy(np.ascontiguousarray(obs.astype(np.uint8))).cuda()
    dm = _device_model(m)
    asym = dict(dm, knots=np.array([0.1, 0.5, 0.8]), q=3)
    assert ta.timestral_forecast(out, xd, od, asym, b, v, x.shape[1], horizon) == ta.E_INVALID
    args = ta.timestral_forecast_args(out, xd, od, dm, b, v, x.shape[1], horizon)
    args.flags = 0  # host pointers are not taken
    import ctypes

    assert ta.load().tsfm_timestral_forecast(ctypes.byref(args)) == ta.E_UNSUPPORTED
    args.flags = ta.DEVICE_PTRS | 8  # no such flag
    assert ta.load().tsfm_timestral_forecast(ctypes.byref(args)) == ta.E_INVALID
    torch.cuda.synchronize()
    assert (out == 0).all()


def _cov_case(seed, b=2, v=1, n_past=1, n_known=2, length=150, horizon=40):
    """A past-only row with a gap, a known-future row with missing future steps and a 0/1
    indicator row (its statistics skipped, no asinh)."""
    m, x, obs = _case(seed, b, v, length)
    rng = np.random.default_rng(seed + 100)
    past = (3 + rng.standard_normal((b, n_past, length))).astype(np.float32)
    past[:, :, 40:55] = np.nan
    steps = np.arange(length + horizon)
    known = np.empty((b, n_known, length + horizon), np.float32)
    for k in range(n_known):
        known[:, k] = np.cos(steps / 5.0 + k) * 4 + 10 if k != 1 else (steps % 7 < 2)
    known[:, 0, length + 3:length + 9] = np.nan
    return m, x, obs, past, known


@pytest.mark.parametrize("horizon,per_shot,max_context,v", [(40, 32, 0, 1), (100, 2, 0, 2), (100, 2, 176, 1)])
def test_timestral_forecast_with_covariates(ta, orc, orc16, gpu_ready, horizon, per_shot, max_context, v):
    """Past-only and known-future covariates (forecaster.zig:57-121, 321-394; model.zig:240-330):
    the window over context and horizon, known rows' whole-window statistics and bidirectional
    time attention, the variate firewalls, role feedback between blocks, and the mirrored pass over
    negated covariates, against the oracle's re-encoding forecast at the reference-derived bar."""
    import torch

    b = 2
    m, x, obs, past, known = _cov_case(41 + v, b, v, horizon=horizon)
    t = x.shape[1]
    out = torch.full((b, v, horizon, m["q"]), -7.0, device="cuda")
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    od = torch.from_numpy(np.ascontiguousarray(obs.astype(np.uint8))).cuda()
    rc = ta.timestral_forecast(out, xd, od, _device_model(m), b, v, t, horizon, max_context=max_context,
                               per_shot=per_shot, past=torch.from_numpy(past).cuda(),
                               known=torch.from_numpy(known).cuda())
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kw = dict(max_context=max_context, per_shot=per_shot)
    rc8, w8 = orc.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, past, known, **kw)
    rc16, w16 = orc16.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, past, known, **kw)
    assert rc8 == 0 and rc16 == 0
    print(f"covariates horizon={horizon} per_shot={per_shot} max_context={max_context} v={v}", flush=True)
    err, bar = _ref.assert_within_reference_bar(got, w8, w16)
    print(f"  err {err:.3g} bar {bar:.3g}", flush=True)
    _, plain = orc16.timestral_forecast(THREADS, m, x, obs, b, v, t, horizon, max_context, per_shot)
    assert _ref.scaled_err(got, plain) > 10 * bar  # the covariates do move the forecast


@pytest.mark.parametrize("max_context", [0, 176])
def test_timestral_cached_decode_with_past_covariates(ta, orc, orc16, gpu_ready, max_context):
    """Past-only covariates keep every encoder token causal in time, so the K/V cache stays exact:
    the cached forecast over several decode blocks equals the re-encoding one (up to f32
    summation order) and both are within the reference-derived bar of the oracle's re-encoding
    forecast; with a known-future row as well the cache is not used (the two calls agree
    exactly)."""
    import torch

    b, v, horizon, per_shot = 2, 2, 100, 2
    m, x, obs, past, known = _cov_case(70 + max_context, b, v, n_past=3, n_known=1, horizon=horizon)
    t = x.shape[1]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731

    def run(kv_cache, **cov):
        out = torch.full((b, v, horizon, m["q"]), -7.0, device="cuda")
        rc = ta.timestral_forecast(out, dev(x), dev(obs.astype(np.uint8)), _device_model(m), b, v, t, horizon,
                                   max_context=max_context, per_shot=per_shot, kv_cache=kv_cache,
                                   **{k: dev(a) for k, a in cov.items()})
        assert rc == ta.OK, ta.last_error()
        torch.cuda.synchronize()
        return out.cpu().numpy()

    cached, full = run(True, past=past), run(False, past=past)
    diff = _ref.scaled_err(cached, full)
    print(f"past covariates, max_context={max_context}: cached vs re-encoded {diff:.3g}", flush=True)
    assert diff < 2e-5
    kw = dict(max_context=max_context, per_shot=per_shot)
    rc8, w8 = orc.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, past, None, **kw)
    rc16, w16 = orc16.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, past, None, **kw)
    assert rc8 == 0 and rc16 == 0
    _ref.assert_within_reference_bar(cached, w8, w16)
    assert np.array_equal(run(True, past=past, known=known), run(False, past=past, known=known))


@pytest.mark.parametrize("v,n_past,n_known", [(1, 8, 8), (2, 12, 10), (1, 16, 16)])
def test_timestral_forecast_many_rows(ta, orc, orc16, gpu_ready, v, n_past, n_known):
    """17, 24 and 33 rows per series (targets and covariates): the variate layers take the
    row-block kernel; against both oracle builds' re-encoding forecasts at the reference-derived
    bar, over two decode blocks."""
    import torch

    b, horizon, per_shot = 2, 40, 2
    m, x, obs, past, known = _cov_case(60 + v + n_past, b, v, n_past=n_past, n_known=n_known, horizon=horizon)
    t = x.shape[1]
    out = torch.full((b, v, horizon, m["q"]), -7.0, device="cuda")
    rc = ta.timestral_forecast(out, torch.from_numpy(x).cuda(), torch.from_numpy(obs.astype(np.uint8)).cuda(),
                               _device_model(m), b, v, t, horizon, per_shot=per_shot,
                               past=torch.from_numpy(past).cuda(), known=torch.from_numpy(known).cuda())
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kw = dict(max_context=0, per_shot=per_shot)
    rc8, w8 = orc.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, past, known, **kw)
    rc16, w16 = orc16.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, past, known, **kw)
    assert rc8 == 0 and rc16 == 0
    err, bar = _ref.assert_within_reference_bar(got, w8, w16)
    print(f"rows {v + n_past + n_known}: err {err:.3g} bar {bar:.3g}", flush=True)


@pytest.mark.parametrize("v,max_context", [(1, 0), (1, 96), (2, 0)])
def test_timestral_forecast_with_categorical_covariates(ta, orc, orc16, gpu_ready, v, max_context):
    """Categorical past and known codes (Covariates.cat_past / .cat_known, forecaster.zig:86-103):
    encoded on the host by the library (target encoding with one variate, raw codes with two),
    appended after the numeric rows, forecast on the device; against both oracle builds' forecasts
    of the oracle-encoded rows at the reference-derived bar."""
    import torch

    b, horizon, per_shot = 2, 40, 2
    m, x, obs, past, known = _cov_case(80 + v, b, v, horizon=horizon)
    t = x.shape[1]
    rng = np.random.default_rng(81)
    cat_past = rng.integers(0, 4, (b, 2, t)).astype(np.float64)
    cat_past[:, 0, 20:30] = np.nan
    cat_known = (np.arange(t + horizon) // 7 % 3).astype(np.float64)[None, None].repeat(b, 0)
    cat_known[:, :, t + 5] = 9.0  # a code the context never had
    out = torch.full((b, v, horizon, m["q"]), -7.0, device="cuda")
    rc = ta.timestral_forecast(out, torch.from_numpy(x).cuda(), torch.from_numpy(obs.astype(np.uint8)).cuda(),
                               _device_model(m), b, v, t, horizon, max_context=max_context, per_shot=per_shot,
                               past=torch.from_numpy(past).cuda(), known=torch.from_numpy(known).cuda(),
                               cat_past=cat_past, cat_known=cat_known)
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    window = max_context or m["context_length"]
    x3, o3 = x.reshape(b, v, t), obs.reshape(b, v, t)
    enc_p = orc.timestral_encode_categorical(cat_past, x3, o3, window)
    enc_k = orc.timestral_encode_categorical(cat_known, x3, o3, window)
    rows_p, rows_k = np.concatenate([past, enc_p], 1), np.concatenate([known, enc_k], 1)
    kw = dict(max_context=max_context, per_shot=per_shot)
    rc8, w8 = orc.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, rows_p, rows_k, **kw)
    rc16, w16 = orc16.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, rows_p, rows_k, **kw)
    assert rc8 == 0 and rc16 == 0
    err, bar = _ref.assert_within_reference_bar(got, w8, w16)
    print(f"categorical v={v} max_context={max_context}: err {err:.3g} bar {bar:.3g}", flush=True)
    _, numeric_only = orc16.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, past, known, **kw)
    assert _ref.scaled_err(got, numeric_only) > 10 * bar  # the categorical rows do move the forecast


@pytest.mark.parametrize("max_context", [0, 176])
def test_timestral_forecast_with_covariates_bf16(ta, orc16, gpu_ready, max_context):
    """TSFM_TIMESTRAL_BF16_ATTN with covariates: the per-row time-attention launches over the bf16
    K/V (two-byte elements, FULL_KEYS known rows, the decoder rows' output offsets), several decode
    blocks with role feedback, with and without the max_context slide, against the 16-lane oracle's
    f32 re-encoding forecast at the half-precision bar (a model in linear space: use_asinh off)."""
    import torch

    b, v, horizon, per_shot = 2, 1, 100, 2
    _, x, obs, past, known = _cov_case(47, b, v, horizon=horizon)
    m = _ref.timestral_model(np.random.default_rng(48), d=128, nh=2, hid=256, use_asinh=False)
    t = x.shape[1]
    outs = {}
    for bf16 in (True, False):
        out = torch.full((b, v, horizon, m["q"]), -7.0, device="cuda")
        rc = ta.timestral_forecast(out, torch.from_numpy(x).cuda(), torch.from_numpy(obs.astype(np.uint8)).cuda(),
                                   _device_model(m), b, v, t, horizon, max_context=max_context, per_shot=per_shot,
                                   past=torch.from_numpy(past).cuda(), known=torch.from_numpy(known).cuda(),
                                   attn_bf16=bf16)
        assert rc == ta.OK, ta.last_error()
        torch.cuda.synchronize()
        outs[bf16] = out.cpu().numpy()
    rc, want = orc16.timestral_forecast_cov(THREADS, m, x, obs, b, v, t, horizon, past, known, max_context=max_context,
                                            per_shot=per_shot)
    assert rc == 0
    err = _ref.scaled_err(outs[True], want)
    print(f"bf16 covariates max_context={max_context}: {err:.3g} (f32 {_ref.scaled_err(outs[False], want):.3g})")
    assert np.isfinite(outs[True]).all()
    assert err < 1e-2, err
    assert _ref.scaled_err(outs[False], want) < err  # the bf16 rounding is what moves the forecast


def test_timestral_forecast_covariate_errors(ta, gpu_ready):
    import torch

    m, x, obs, past, known = _cov_case(45)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    od = torch.from_numpy(np.ascontiguousarray(obs.astype(np.uint8))).cuda()
    out = torch.zeros((2, 1, 40, m["q"]), device="cuda")
    a = ta.timestral_forecast_args(out, xd, od, _device_model(m), 2, 1, x.shape[1], 40,
                                   known=torch.from_numpy(known).cuda())
    a.known = None  # a count without its array
    assert ta.load().tsfm_timestral_forecast(ta.ctypes.byref(a)) == ta.E_INVALID
    big = torch.zeros((2, ta.VARIATE_MAX_ROWS, x.shape[1] + 40), device="cuda")
    rc = ta.timestral_forecast(out, xd, od, _device_model(m), 2, 1, x.shape[1], 40, known=big)
    assert rc == ta.E_UNSUPPORTED  # 1 target + 256 covariate rows: more than the kernels' 256
    # config.zig:49-70: a schedule of time ops only cannot route a known future to the targets
    # (error.KnownCovariatesUnsupported); past-only covariates still run.
    rng = np.random.default_rng(46)
    tm = _device_model(_ref.timestral_model(rng, d=128, nh=2, hid=256, schedule=("time", "time")))
    kd, pd = torch.from_numpy(known).cuda(), torch.from_numpy(past).cuda()
    assert ta.timestral_forecast(out, xd, od, tm, 2, 1, x.shape[1], 40, known=kd) == ta.E_UNSUPPORTED
    assert "KnownCovariatesUnsupported" in ta.last_error()
    assert ta.timestral_forecast(out, xd, od, tm, 2, 1, x.shape[1], 40, past=pd) == ta.OK, ta.last_error()
