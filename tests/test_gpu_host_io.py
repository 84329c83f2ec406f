"""TSFM_FORECAST_HOST_IO: the four forecast entry points with their per-call arrays (inputs,
observed, covariates, out) in host memory and the weights on the device, as a host caller that
registered its weights once (tsfm_weight_register) makes them. The call stages the arrays through
the calling thread's stream and returns with out written; the result is the device-pointer call's,
bit for bit (the same kernels on the same inputs)."""
import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu


def test_bolt_forecast_host_io(ta, gpu_ready):
    import torch

    import test_gpu_bolt_forward as T

    nh, d_ff, out_w, n, length = 2, 256, 48, 5, 150
    s = T._setup(61, n, (length + 15) // 16, nh, d_ff, 2, 2, out_w)
    ctx = T._forecast_ctx(np.random.default_rng(3), n, length)
    want = T._forecast(ta, s, ctx, n, length, nh, d_ff, out_w)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    out = np.full((n, out_w), -9.0, np.float32)
    rc = ta.bolt_forecast(out, ctx, length, cu(s["reg"]), cu(s["start"]), cu(s["table"]),
                          [{k: cu(v) for k, v in ly.items()} for ly in s["enc"]], cu(s["ef"]),
                          [{k: cu(v) for k, v in ly.items()} for ly in s["dec"]], cu(s["df"]),
                          {k: cu(v) for k, v in s["ie"].items()}, {k: cu(v) for k, v in s["oe"].items()}, n, s["d"],
                          nh, d_ff, 1e-6)
    assert rc == ta.OK, ta.last_error()
    assert np.array_equal(out, want)


def test_chronos2_forecast_host_io(ta, orc, gpu_ready):
    import torch

    import test_gpu_encoder as T

    nh, d_ff, n, tsc, length, horizon = 2, 256, 4, 8192.0, 150, 20
    c = T._forecast_case(orc, 7, length, horizon, nh, d_ff)
    rng = np.random.default_rng(8)
    x = (5.0 + 3.0 * rng.standard_normal((n, length))).astype(np.float32)
    x[rng.random((n, length)) < 0.1] = np.nan
    want = T._c2_forecast(ta, c, x, n, length, horizon, nh, d_ff, True, tsc)
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    out = np.full((n, horizon, c["q"]), -9.0, np.float32)
    rc = ta.chronos2_forecast(out, x, length, horizon, cu(c["reg"]), cu(c["cos"]), cu(c["sin"]),
                              [{k: cu(v) for k, v in ly.items()} for ly in c["layers"]], cu(c["fn"]),
                              {k: cu(v) for k, v in c["ie"].items()}, {k: cu(v) for k, v in c["oe"].items()}, n,
                              c["d"], nh, d_ff, 1e-6, time_scale=tsc, arcsinh=True)
    assert rc == ta.OK, ta.last_error()
    assert np.array_equal(out, want)


def test_bolt_forecast_horizon_host_io(ta, gpu_ready):
    import test_gpu_bolt_horizon as T

    w = T._small()
    x = T._series(9, 3, 130)
    horizon, P, max_ctx = 33, 16, 64
    want = T._gpu_horizon(ta, w, x, horizon, P, max_ctx)
    dv = T._device(w)
    out = np.full((x.shape[0], horizon, T.LEVELS.size), -7.0, np.float32)
    rc = ta.bolt_forecast_horizon(out, np.ascontiguousarray(x), horizon, dv["reg"], dv["dec_start"], dv["rel_table"],
                                  dv["enc"], dv["enc_final_norm"], dv["dec"], dv["dec_final_norm"], dv["ie"], dv["oe"],
                                  w["d_model"], w["heads"], w["d_ff"], w["eps"], T.LEVELS, P, max_ctx)
    assert rc == ta.OK, ta.last_error()
    assert np.array_equal(out, want)


@pytest.mark.parametrize("covariates", [False, True])
def test_timestral_forecast_host_io(ta, gpu_ready, covariates):
    import torch

    import test_gpu_timestral as T

    b, v, horizon = 2, 1, 40
    m, x, obs, past, known = T._cov_case(90, b, v, horizon=horizon)
    t = x.shape[1]
    cat = np.random.default_rng(91).integers(0, 3, (b, 1, t)).astype(np.float64) if covariates else None
    kw = dict(per_shot=2, kv_cache=True)
    if covariates:
        kw.update(past=past, known=known, cat_past=cat)
    dm = T._device_model(m)
    outs = []
    for host in (False, True):
        conv = (lambda a: np.ascontiguousarray(a)) if host else (lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda())
        args = {k: (conv(val) if isinstance(val, np.ndarray) and k in ("past", "known") else val) for k, val in kw.items()}
        out = np.full((b, v, horizon, m["q"]), -7.0, np.float32) if host else torch.full((b, v, horizon, m["q"]), -7.0,
                                                                                          device="cuda")
        rc = ta.timestral_forecast(out, conv(x), conv(obs.astype(np.uint8)), dm, b, v, t, horizon, **args)
        assert rc == ta.OK, ta.last_error()
        torch.cuda.synchronize()
        outs.append(out if host else out.cpu().numpy())
    assert np.isfinite(outs[1]).all()
    assert np.array_equal(outs[0], outs[1])
