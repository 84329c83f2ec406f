"""GPU parity of the Chronos-Bolt model forward (tsfm_bolt_forward: input embedding,
[patches; REG], the T5 encoder with the relative position bias, the one-token decoder with
cross-attention, the output head) against the oracle's restatement of the forecaster's chunk
(src/chronos_bolt/forecaster.zig:199-213, Model.encode/decode src/chronos_bolt/model.zig:210-308)
and against the same computation in float64, through the C ABI.

Bar: _ref.reference_bar against the oracle's 16-lane (AVX-512) build: twice the larger of the
reference's own cross-host spread (its 8-lane against its 16-lane build) and its distance from
float64 where a float64 evaluation exists, never tighter than 1e-5. Covered: padded and
all-valid patches, the Chronos-Bolt-small shape (d 512, 8 heads, d_ff 2048, 32 patches + REG,
9 quantiles x 64 steps), host and device pointers (same bits); the whole forecast
(src/chronos_bolt/forecaster.zig:128-220: instance norm, left-padded [values, mask] patches, the
model, the inverse norm) on whole, padded and sub-patch contexts with missing values, strided rows,
a constant and an all-missing series.
"""
import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu

THREADS = 16


def _setup(seed, b, n_patch, nh, d_ff, n_enc, n_dec, out, ps=16, all_valid=False):
    rng = np.random.default_rng(seed)
    d = inner = nh * 64
    feats = rng.standard_normal((b * n_patch, 2 * ps)).astype(np.float32)
    pv = np.ones((b, n_patch), np.uint8) if all_valid else (rng.random((b, n_patch)) < 0.8).astype(np.uint8)
    reg, start = (rng.standard_normal(d).astype(np.float32) for _ in range(2))
    table = _ref.t5_bias_table(rng, 32, nh)
    enc, dec = _ref.bolt_layers(rng, n_enc, n_dec, d, inner, d_ff)
    ef, df = ((1 + 0.1 * rng.standard_normal(d)).astype(np.float32) for _ in range(2))
    ie, oe = _ref.resblock(rng, 2 * ps, d_ff, d), _ref.resblock(rng, d, d_ff, out)
    return dict(feats=feats, pv=pv, reg=reg, start=start, table=table, enc=enc, dec=dec, ef=ef, df=df, ie=ie, oe=oe,
                d=d)


def _run(ta, s, b, n_patch, nh, d_ff, out):
    raw = np.full((b, out), -9.0, np.float32)
    rc = ta.bolt_forward(raw, s["feats"], s["pv"], s["reg"], s["start"], s["table"], s["enc"], s["ef"], s["dec"],
                         s["df"], s["ie"], s["oe"], b, n_patch, s["d"], nh, d_ff, 1e-6)
    assert rc == ta.OK, ta.last_error()
    return raw


def _oracle(orc, s, b, n_patch, nh, d_ff, out):
    want = np.zeros((b, out), np.float32)
    orc.bolt_model_forward(THREADS, want, s["feats"], s["pv"], s["reg"], s["start"], s["table"], 32, 128, b, n_patch,
                           s["d"], nh, 64, d_ff, s["enc"], s["ef"], s["dec"], s["df"], 1e-6, s["ie"], s["oe"])
    return want


def _exact(orc, s, b, n_patch, nh):
    bias = orc.position_bias(s["table"], n_patch + 1, nh, 32, 128)
    return _ref.bolt_model_forward_f64(s["feats"], s["pv"], s["reg"], s["start"], bias, b, n_patch, nh, s["enc"],
                                       s["ef"], s["dec"], s["df"], 1e-6, s["ie"], s["oe"])


@pytest.mark.parametrize("all_valid", [False, True])
def test_bolt_forward_matches_oracle_and_f64(ta, orc, orc16, gpu_ready, all_valid):
    b, n_patch, nh, d_ff, out = 4, 20, 2, 256, 48
    s = _setup(50 + all_valid, b, n_patch, nh, d_ff, 2, 2, out, all_valid=all_valid)
    raw = _run(ta, s, b, n_patch, nh, d_ff, out)
    w8, w16 = (_oracle(o_, s, b, n_patch, nh, d_ff, out) for o_ in (orc, orc16))
    _ref.assert_within_reference_bar(raw, w8, w16, _exact(orc, s, b, n_patch, nh))


@pytest.mark.parametrize("b,n_dec", [(20, 3), (5, 3)])
def test_bolt_forward_decoder_paths(ta, orc, orc16, gpu_ready, b, n_dec):
    """The decoder's two forms against the oracle: more than 16 series (row norms as launches or in
    the producing product) and at most 16 (the 16-row products normalise their inputs on load);
    an odd number of decoder layers, so the last cross-attention K/V product runs one layer alone
    (the others two layers per four-output product)."""
    n_patch, nh, d_ff, out = 12, 2, 256, 32
    s = _setup(90 + b, b, n_patch, nh, d_ff, 2, n_dec, out)
    raw = _run(ta, s, b, n_patch, nh, d_ff, out)
    w8, w16 = (_oracle(o_, s, b, n_patch, nh, d_ff, out) for o_ in (orc, orc16))
    _ref.assert_within_reference_bar(raw, w8, w16, _exact(orc, s, b, n_patch, nh))


def test_bolt_forward_small_shape(ta, orc, orc16, gpu_ready):
    """Chronos-Bolt-small: d_model 512, 8 heads of 64, d_ff 2048, 6 + 6 layers, 32 patches + REG,
    9 quantiles x 64 steps; 16 series. Twelve f32 layers: every evaluation drifts from the exact
    result with depth, the reference's own included; the bar follows it."""
    b, n_patch, nh, d_ff, out = 16, 32, 8, 2048, 9 * 64
    s = _setup(7, b, n_patch, nh, d_ff, 6, 6, out)
    raw = _run(ta, s, b, n_patch, nh, d_ff, out)
    w8, w16 = (_oracle(o_, s, b, n_patch, nh, d_ff, out) for o_ in (orc, orc16))
    exact = _exact(orc, s, b, n_patch, nh)
    assert _ref.scaled_err(w16, exact) < 5e-4
    _ref.assert_within_reference_bar(raw, w8, w16, exact)
    _ref.assert_no_further_from_exact(raw, w8, w16, exact)


def test_bolt_forward_device_pointers_match_host(ta, orc, gpu_ready):
    import torch

    b, n_patch, nh, d_ff, out = 3, 12, 2, 128, 32
    s = _setup(9, b, n_patch, nh, d_ff, 2, 1, out)
    host = _run(ta, s, b, n_patch, nh, d_ff, out)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    raw = torch.zeros((b, out), device="cuda")
    rc = ta.bolt_forward(raw, cu(s["feats"]), cu(s["pv"]), cu(s["reg"]), cu(s["start"]), cu(s["table"]),
                         [{k: cu(v) for k, v in ly.items()} for ly in s["enc"]], cu(s["ef"]),
                         [{k: cu(v) for k, v in ly.items()} for ly in s["dec"]], cu(s["df"]),
                         {k: cu(v) for k, v in s["ie"].items()}, {k: cu(v) for k, v in s["oe"].items()}, b, n_patch,
                         s["d"], nh, d_ff, 1e-6, keys_all_valid=bool(s["pv"].all()))
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), host)


# ---- the whole forecast: instance norm and patching on the device, the model, the inverse norm ----


def _forecast_ctx(rng, n, length, nan_frac=0.1):
    ctx = (3.0 + 2.0 * rng.standard_normal((n, length))).astype(np.float32)
    ctx[rng.random((n, length)) < nan_frac] = np.nan
    return ctx


def _forecast(ta, s, ctx, n, length, nh, d_ff, out_w, stride=None, offset=0):
    import torch

    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = torch.full((n, out_w), -9.0, device="cuda")
    rc = ta.bolt_forecast(out, cu(ctx), length, cu(s["reg"]), cu(s["start"]), cu(s["table"]),
                          [{k: cu(v) for k, v in ly.items()} for ly in s["enc"]], cu(s["ef"]),
                          [{k: cu(v) for k, v in ly.items()} for ly in s["dec"]], cu(s["df"]),
                          {k: cu(v) for k, v in s["ie"].items()}, {k: cu(v) for k, v in s["oe"].items()}, n, s["d"],
                          nh, d_ff, 1e-6, stride=stride, offset=offset)
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _forecast_oracle(orc, s, ctx, length, n, nh, d_ff, out_w, stride=None, offset=0):
    want = np.zeros((n, out_w), np.float32)
    orc.bolt_forecast(THREADS, want, ctx, stride or length, offset, length, n, 16, 1e-5, s["reg"], s["start"],
                      s["table"], 32, 128, s["d"], nh, 64, d_ff, s["enc"], s["ef"], s["dec"], s["df"], 1e-6, s["ie"],
                      s["oe"])
    return want


@pytest.mark.parametrize("length", [160, 150, 7])
def test_bolt_forecast_matches_oracle(ta, orc, orc16, gpu_ready, length):
    """Context lengths that fill whole patches (160), that need left padding (150: 10 missing steps
    before the first patch) and that are shorter than one patch (7), with ~10 % missing values. The
    instance norm and patching are exact restatements, so the bar is the model forward's."""
    nh, d_ff, out_w, n = 2, 256, 48, 5
    n_patch = (length + 15) // 16
    s = _setup(60 + length, n, n_patch, nh, d_ff, 2, 2, out_w)
    ctx = _forecast_ctx(np.random.default_rng(length), n, length)
    got = _forecast(ta, s, ctx, n, length, nh, d_ff, out_w)
    w8, w16 = (_forecast_oracle(o_, s, ctx, length, n, nh, d_ff, out_w) for o_ in (orc, orc16))
    assert np.isfinite(got).all()
    _ref.assert_within_reference_bar(got, w8, w16)


def test_bolt_forecast_strided_rows_and_degenerate_series(ta, orc, orc16, gpu_ready):
    """Rows read at a stride and offset from a wider buffer; one series constant (zero spread: the
    scale becomes norm_eps, so every forecast is the constant plus 1e-5 times the raw output) and one
    entirely missing (loc 0, scale 1: the forecast is the raw output of all-zero features)."""
    nh, d_ff, out_w, n, length, stride, offset = 2, 128, 32, 4, 40, 57, 9
    s = _setup(71, n, 3, nh, d_ff, 1, 1, out_w)
    rng = np.random.default_rng(3)
    buf = (1.0 + rng.standard_normal(n * stride + offset)).astype(np.float32)
    rows = lambda: [buf[i * stride + offset:][:length] for i in range(n)]
    rows()[1][:] = 4.25
    rows()[2][:] = np.nan
    rows()[3][::3] = np.nan
    got = _forecast(ta, s, buf, n, length, nh, d_ff, out_w, stride=stride, offset=offset)
    w8, w16 = (_forecast_oracle(o_, s, buf, length, n, nh, d_ff, out_w, stride=stride, offset=offset)
               for o_ in (orc, orc16))
    _ref.assert_within_reference_bar(got, w8, w16)
    assert np.abs(got[1] - 4.25).max() < 1e-3
    # The all-missing series: features are all zero and every context patch is masked, so its
    # forecast is the model forward of zero features with no valid patch (a batch of one here, so
    # the products may split their sums differently: 5e-5, the width of a few f32 roundings at
    # this depth).
    feats = np.zeros((3, 32), np.float32)
    raw = np.zeros((1, out_w), np.float32)
    rc = ta.bolt_forward(raw, feats, np.zeros((1, 3), np.uint8), s["reg"], s["start"], s["table"], s["enc"], s["ef"],
                         s["dec"], s["df"], s["ie"], s["oe"], 1, 3, s["d"], nh, d_ff, 1e-6)
    assert rc == ta.OK, ta.last_error()
    assert _ref.scaled_err(got[2:3], raw) <= 5e-5


def test_bolt_small_forecast_end_to_end_workload(ta, orc, orc16, gpu_ready):
    """The end-to-end configuration itself: Chronos-Bolt-small (d 512, 8 heads, d_ff 2048, 6 + 6
    layers, 9 quantiles x 64), 16 series of 512 steps, each a period-24 sinusoid of amplitude 10 plus
    a linear trend plus N(0, 1) noise from seed 0 with 2 % of the values NaN, horizon 64, through
    tsfm_bolt_forecast, against the oracle's forecaster chunk (src/chronos_bolt/forecaster.zig:128-220)."""
    from tsfm_attn import workloads

    w = workloads.bolt_forward()
    a, m = w.arrays, w.meta
    s = dict(reg=a["reg"], start=a["dec_start"], table=a["rel_table"], enc=m["enc"], ef=a["enc_final_norm"],
             dec=m["dec"], df=a["dec_final_norm"], ie=m["ie"], oe=m["oe"], d=m["d_model"])
    ctx = np.ascontiguousarray(a["ctx"])
    n, length = ctx.shape
    assert (n, length, m["out"]) == (16, 512, 9 * 64) and np.isnan(ctx).mean() > 0.01
    got = _forecast(ta, s, ctx, n, length, w.H, m["d_ff"], m["out"])
    w8, w16 = (_forecast_oracle(o_, s, ctx, length, n, w.H, m["d_ff"], m["out"]) for o_ in (orc, orc16))
    assert np.isfinite(got).all()
    _ref.assert_within_reference_bar(got, w8, w16)
