"""GPU parity of the Chronos-2 encoder stack (tsfm_chronos2_encode) and of the model part of the
forecaster (tsfm_chronos2_forward: input embedding, [context; REG; future], encoder, output head)
against the oracle's restatements of Model.encode (src/chronos2/model.zig:144-206) and of runChunk
(src/chronos2/forecaster.zig:155-183), and against the same computations in float64, through the
C ABI.

A stack of layers composes many f32 reductions: the GPU's and the oracle's summation orders
differ, and both differ from exact arithmetic by about as much. The bar is _ref.reference_bar:
against the oracle's 16-lane (AVX-512) build, twice the larger of the reference's own cross-host
spread (its 8-lane build against its 16-lane build) and the reference's distance from float64
where a float64 evaluation exists, and never tighter than 1e-5. Covered: scale 1/8 and the
model's 1.0, padded and all-valid keys (FULL and KEYS_ADDITIVE masks give the same result when
every key is valid), no layers (final norm only), host and device pointers (same bits), a
Chronos-2-base shaped run (d 768, 12 heads, d_ff 3072, 577 tokens), and twelve layers.
The whole forecast (tsfm_chronos2_forecast: instance norm, time-encoded
patch features, the model, inverse scaling) against the oracle's runChunk on whole, padded and
sub-patch contexts, cut horizons, asinh space on and off, strided rows, a constant and an
all-missing series.
"""
import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu

THREADS = 16


def _setup(seed, b, seq, nh, d_ff, n_layers, pad=True):
    rng = np.random.default_rng(seed)
    d = nh * 64
    x = rng.standard_normal((b * seq, d)).astype(np.float32)
    kv = _ref.left_pad_valid(rng, b, seq, seq // 4, tail_valid=2) if pad else np.ones((b, seq), np.uint8)
    layers = _ref.chronos2_layers(rng, n_layers, d, d_ff)
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return x, kv, layers, fn, d


def _oracle(orc, x, kv, layers, fn, b, seq, d, nh, d_ff, eps, cos_t, sin_t, scale):
    want = x.copy()
    orc.chronos2_encode(THREADS, want, kv.ravel().copy(), b, seq, d, nh, 64, d_ff, layers, fn, eps, cos_t, sin_t,
                        scale)
    return want


def _both(orc, orc16, *args):
    """The oracle's 8-lane and 16-lane results of the same call."""
    return _oracle(orc, *args), _oracle(orc16, *args)


@pytest.mark.parametrize("scale", [0.125, 1.0])
@pytest.mark.parametrize("pad", [True, False])
def test_encode_matches_oracle_and_f64(ta, orc, orc16, gpu_ready, scale, pad):
    b, seq, nh, d_ff, n_layers, eps = 3, 45, 2, 256, 3, 1e-6
    x, kv, layers, fn, d = _setup(int(scale * 8) + 10 * pad, b, seq, nh, d_ff, n_layers, pad)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    got = x.copy()
    rc = ta.chronos2_encode(got, kv, cos_t, sin_t, layers, fn, b, seq, d, nh, d_ff, eps, scale=scale)
    assert rc == ta.OK, ta.last_error()
    w8, w16 = _both(orc, orc16, x, kv, layers, fn, b, seq, d, nh, d_ff, eps, cos_t, sin_t, scale)
    exact = _ref.chronos2_encode_f64(x, kv, b, seq, nh, layers, fn, eps, cos_t, sin_t, scale)
    _ref.assert_within_reference_bar(got, w8, w16, exact)
    if not pad:  # every key valid: the KEYS_ADDITIVE mask (keys_all_valid=False) gives the same bits
        again = x.copy()
        rc = ta.chronos2_encode(again, kv, cos_t, sin_t, layers, fn, b, seq, d, nh, d_ff, eps, scale=scale,
                                keys_all_valid=False)
        assert rc == ta.OK, ta.last_error()
        assert _ref.scaled_err(again, got) <= 1e-6


def test_encode_without_layers_is_the_final_norm(ta, orc, gpu_ready):
    b, seq, nh = 2, 17, 1
    x, kv, _, fn, d = _setup(3, b, seq, nh, 64, 0)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    got = x.copy()
    assert ta.chronos2_encode(got, kv, cos_t, sin_t, [], fn, b, seq, d, nh, 64, 1e-6) == ta.OK, ta.last_error()
    assert _ref.scaled_err(got, _ref.rms_norm_f64(x, fn, 1e-6)) <= 2e-6


def test_encode_device_pointers_match_host(ta, orc, gpu_ready):
    import torch

    b, seq, nh, d_ff, n_layers, eps = 2, 33, 2, 128, 2, 1e-6
    x, kv, layers, fn, d = _setup(21, b, seq, nh, d_ff, n_layers)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    host = x.copy()
    assert ta.chronos2_encode(host, kv, cos_t, sin_t, layers, fn, b, seq, d, nh, d_ff, eps) == ta.OK, ta.last_error()
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    dl = [{k: cu(v) for k, v in ly.items()} for ly in layers]
    xd = cu(x)
    rc = ta.chronos2_encode(xd, cu(kv), cu(cos_t), cu(sin_t), dl, cu(fn), b, seq, d, nh, d_ff, eps,
                            keys_all_valid=bool(kv.all()))
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(xd.cpu().numpy(), host)


def test_encode_chronos2_base_shape(ta, orc, orc16, gpu_ready):
    """d_model 768, 12 heads, d_ff 3072 over 577 tokens (512 context patches, REG, 64 future), two
    layers of the model's scale 1.0."""
    b, seq, nh, d_ff, n_layers, eps = 2, 577, 12, 3072, 2, 1e-6
    x, kv, layers, fn, d = _setup(5, b, seq, nh, d_ff, n_layers)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    got = x.copy()
    rc = ta.chronos2_encode(got, kv, cos_t, sin_t, layers, fn, b, seq, d, nh, d_ff, eps, scale=1.0)
    assert rc == ta.OK, ta.last_error()
    w8, w16 = _both(orc, orc16, x, kv, layers, fn, b, seq, d, nh, d_ff, eps, cos_t, sin_t, 1.0)
    _ref.assert_within_reference_bar(got, w8, w16)


def test_encode_twelve_layers_drift_like_the_oracle(ta, orc, orc16, gpu_ready):
    """Twelve Chronos-2-base layers at the model's scale 1.0: every f32 evaluation drifts from the
    exact result with depth, the reference's own included; the bar follows it."""
    b, seq, nh, d_ff, n_layers, eps = 1, 145, 12, 3072, 12, 1e-6
    x, kv, layers, fn, d = _setup(12, b, seq, nh, d_ff, n_layers)
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    got = x.copy()
    rc = ta.chronos2_encode(got, kv, cos_t, sin_t, layers, fn, b, seq, d, nh, d_ff, eps, scale=1.0)
    assert rc == ta.OK, ta.last_error()
    w8, w16 = _both(orc, orc16, x, kv, layers, fn, b, seq, d, nh, d_ff, eps, cos_t, sin_t, 1.0)
    exact = _ref.chronos2_encode_f64(x, kv, b, seq, nh, layers, fn, eps, cos_t, sin_t, 1.0)
    assert _ref.scaled_err(w16, exact) < 5e-4  # the f32 reference path itself, for scale
    _ref.assert_within_reference_bar(got, w8, w16, exact)
    _ref.assert_no_further_from_exact(got, w8, w16, exact)


# ---- the model part of the Chronos-2 forecaster: embedding, encoder, output head ------------------


def _forward_setup(seed, b, n_ctx, n_out, nh, d_ff, n_layers, ps=16, q=3):
    rng = np.random.default_rng(seed)
    d = nh * 64
    feats = rng.standard_normal((b * n_ctx, 3 * ps)).astype(np.float32)
    fut = rng.standard_normal((b * n_out, 3 * ps)).astype(np.float32)
    cv = (rng.random((b, n_ctx)) < 0.8).astype(np.uint8)
    reg = rng.standard_normal(d).astype(np.float32)
    layers = _ref.chronos2_layers(rng, n_layers, d, d_ff)
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ie, oe = _ref.resblock(rng, 3 * ps, d_ff, d), _ref.resblock(rng, d, d_ff, q * ps)
    return feats, fut, cv, reg, layers, fn, ie, oe, d


@pytest.mark.parametrize("b,n_ctx,n_out", [(3, 20, 4), (2, 64, 8)])
def test_forward_matches_oracle_and_f64(ta, orc, orc16, gpu_ready, b, n_ctx, n_out):
    nh, d_ff, n_layers, eps, q, ps = 2, 256, 2, 1e-6, 3, 16
    feats, fut, cv, reg, layers, fn, ie, oe, d = _forward_setup(b + n_ctx, b, n_ctx, n_out, nh, d_ff, n_layers)
    seq = n_ctx + 1 + n_out
    cos_t, sin_t = orc.chronos2_rope_tables(seq, 64, 10000.0)
    raw = np.full((b * n_out, q * ps), -9.0, np.float32)
    rc = ta.chronos2_forward(raw, feats, fut, cv, reg, cos_t, sin_t, layers, fn, ie, oe, b, n_ctx, n_out, d, nh, d_ff,
                             eps)
    assert rc == ta.OK, ta.last_error()
    outs = []
    for o_ in (orc, orc16):
        want = np.zeros_like(raw)
        o_.chronos2_model_forward(THREADS, want, feats, fut, cv, reg, b, n_ctx, n_out, d, nh, 64, d_ff, layers, fn, eps,
                                  cos_t, sin_t, 1.0, ie, oe)
        outs.append(want)
    exact = _ref.chronos2_model_forward_f64(feats, fut, cv, reg, b, n_ctx, n_out, nh, layers, fn, eps, cos_t, sin_t,
                                            1.0, ie, oe)
    _ref.assert_within_reference_bar(raw, *outs, exact)


def test_forward_device_pointers_match_host(ta, orc, gpu_ready):
    import torch

    b, n_ctx, n_out, nh, d_ff, eps, q, ps = 2, 30, 5, 2, 128, 1e-6, 3, 16
    feats, fut, cv, reg, layers, fn, ie, oe, d = _forward_setup(77, b, n_ctx, n_out, nh, d_ff, 2)
    cos_t, sin_t = orc.chronos2_rope_tables(n_ctx + 1 + n_out, 64, 10000.0)
    host = np.zeros((b * n_out, q * ps), np.float32)
    rc = ta.chronos2_forward(host, feats, fut, cv, reg, cos_t, sin_t, layers, fn, ie, oe, b, n_ctx, n_out, d, nh,
                             d_ff, eps)
    assert rc == ta.OK, ta.last_error()
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    raw = torch.zeros((b * n_out, q * ps), device="cuda")
    rc = ta.chronos2_forward(raw, cu(feats), cu(fut), cu(cv), cu(reg), cu(cos_t), cu(sin_t),
                             [{k: cu(v) for k, v in ly.items()} for ly in layers], cu(fn),
                             {k: cu(v) for k, v in ie.items()}, {k: cu(v) for k, v in oe.items()}, b, n_ctx, n_out, d,
                             nh, d_ff, eps, keys_all_valid=bool(cv.all()))
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), host)


# ---- the whole Chronos-2 forecast: preparation and inverse scaling on the device around the model -


def _forecast_case(orc, seed, length, horizon, nh=2, d_ff=256, n_layers=2, ps=16, q=3):
    rng = np.random.default_rng(seed)
    d = nh * 64
    reg = rng.standard_normal(d).astype(np.float32)
    layers = _ref.chronos2_layers(rng, n_layers, d, d_ff)
    fn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    ie, oe = _ref.resblock(rng, 3 * ps, d_ff, d), _ref.resblock(rng, d, d_ff, q * ps)
    n_ctx, n_out = (length + ps - 1) // ps, (horizon + ps - 1) // ps
    cos_t, sin_t = orc.chronos2_rope_tables(n_ctx + 1 + n_out, 64, 10000.0)
    return dict(reg=reg, layers=layers, fn=fn, ie=ie, oe=oe, d=d, cos=cos_t, sin=sin_t, q=q)


def _c2_forecast(ta, c, inputs, n, length, horizon, nh, d_ff, arcsinh, tsc, stride=None, start=0):
    import torch

    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = torch.full((n, horizon, c["q"]), -9.0, device="cuda")
    rc = ta.chronos2_forecast(out, cu(inputs), length, horizon, cu(c["reg"]), cu(c["cos"]), cu(c["sin"]),
                              [{k: cu(v) for k, v in ly.items()} for ly in c["layers"]], cu(c["fn"]),
                              {k: cu(v) for k, v in c["ie"].items()}, {k: cu(v) for k, v in c["oe"].items()}, n,
                              c["d"], nh, d_ff, 1e-6, stride=stride, start=start, time_scale=tsc, arcsinh=arcsinh)
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _c2_forecast_oracle(orc, c, inputs, n, length, horizon, nh, d_ff, arcsinh, tsc, stride=None, start=0):
    want = np.zeros((n, horizon, c["q"]), np.float32)
    orc.chronos2_forecast(THREADS, want, inputs, stride or length, start, length, n, 16, horizon, tsc, arcsinh,
                          c["reg"], c["d"], nh, 64, d_ff, c["layers"], c["fn"], 1e-6, c["cos"], c["sin"], 1.0, c["ie"],
                          c["oe"])
    return want


@pytest.mark.parametrize("length,horizon,arcsinh", [(160, 64, True), (150, 20, True), (9, 16, False)])
def test_chronos2_forecast_matches_oracle(ta, orc, orc16, gpu_ready, length, horizon, arcsinh):
    """Whole patches (160), left padding (150) and less than one patch (9); horizons that fill and
    that cut the last future patch; the model's asinh space on and off; ~10 % missing values."""
    nh, d_ff, n, tsc = 2, 256, 4, 8192.0
    c = _forecast_case(orc, length + horizon, length, horizon, nh, d_ff)
    rng = np.random.default_rng(length)
    x = (5.0 + 3.0 * rng.standard_normal((n, length))).astype(np.float32)
    x[rng.random((n, length)) < 0.1] = np.nan
    got = _c2_forecast(ta, c, x, n, length, horizon, nh, d_ff, arcsinh, tsc)
    w8, w16 = (_c2_forecast_oracle(o_, c, x, n, length, horizon, nh, d_ff, arcsinh, tsc) for o_ in (orc, orc16))
    assert np.isfinite(got).all()
    _ref.assert_within_reference_bar(got, w8, w16)


def test_chronos2_forecast_strided_rows_and_degenerate_series(ta, orc, orc16, gpu_ready):
    """Rows at a stride and start offset in a wider buffer (as forecast() reads the last
    context_length steps of each (b, t_in) row); a constant series (scale 1e-5) and an all-missing
    one (loc 0, scale 1, no valid context patch: only REG and the future patches are attended)."""
    nh, d_ff, n, length, horizon, stride, start, tsc = 2, 128, 4, 48, 30, 70, 22, 8192.0
    c = _forecast_case(orc, 5, length, horizon, nh, d_ff, n_layers=1)
    rng = np.random.default_rng(11)
    buf = (1.0 + rng.standard_normal(n * stride)).astype(np.float32)
    rows = lambda: [buf[i * stride + start:][:length] for i in range(n)]
    rows()[1][:] = -3.5
    rows()[2][:] = np.nan
    rows()[3][1::4] = np.nan
    got = _c2_forecast(ta, c, buf, n, length, horizon, nh, d_ff, True, tsc, stride=stride, start=start)
    w8, w16 = (_c2_forecast_oracle(o_, c, buf, n, length, horizon, nh, d_ff, True, tsc, stride=stride, start=start)
               for o_ in (orc, orc16))
    assert np.isfinite(got).all()
    _ref.assert_within_reference_bar(got, w8, w16)


def test_chronos2_base_forecast_at_the_metric_shape(ta, orc, orc16, gpu_ready):
    """The workload behind the benchmark's series-forecasts/s: the Chronos-2-base forecast of 64
    series x 8192 raw steps (oldest 0-25 % missing, 2 % of the rest) with horizon 1024, 12 layers of
    d_model 768, 12 heads, d_ff 3072, 21 quantiles, asinh space. All 64 series run on the device in
    one call, as the benchmark's step does; six of them (the least and most padded and four spread
    over the batch) are checked against both oracle builds at the reference-derived bar."""
    import torch
    from tsfm_attn import workloads

    w = workloads.chronos2_forecast()
    a, m = w.arrays, w.meta
    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()
    d, F, T, hz, q = m["d_model"], m["d_ff"], m["context"], m["horizon"], m["quantiles"]
    out = torch.full((w.B, hz, q), -9.0, device="cuda")
    rc = ta.chronos2_forecast(out, cu(a["ctx"]), T, hz, cu(a["reg"]), cu(a["rope_cos"]), cu(a["rope_sin"]),
                              [{k: cu(v) for k, v in ly.items()} for ly in m["layers"]], cu(a["final_norm"]),
                              {k: cu(v) for k, v in m["ie"].items()}, {k: cu(v) for k, v in m["oe"].items()}, w.B, d,
                              w.H, F, m["eps"], time_scale=m["time_scale"], arcsinh=True)
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    lead = np.isnan(a["ctx"]).argmin(axis=1)  # leading missing steps of each series
    pick = sorted({int(lead.argmin()), int(lead.argmax()), 9, 27, 40, 63})
    ctx = np.ascontiguousarray(a["ctx"][pick])
    outs = []
    for o_ in (orc, orc16):
        want = np.zeros((len(pick), hz, q), np.float32)
        o_.chronos2_forecast(THREADS, want, ctx, T, 0, T, len(pick), m["patch"], hz, m["time_scale"], True, a["reg"], d,
                             w.H, 64, F, m["layers"], a["final_norm"], m["eps"], a["rope_cos"], a["rope_sin"], 1.0,
                             m["ie"], m["oe"])
        outs.append(want)
    err, bar = _ref.assert_within_reference_bar(got[pick], *outs)
    print(f"series {pick}: error {err:.3e}, bar {bar:.3e}")
