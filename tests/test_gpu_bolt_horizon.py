"""GPU parity of Chronos-Bolt forecaster.forecast for any horizon (tsfm_bolt_forecast_horizon,
src/chronos_bolt/forecaster.zig:22-92) and of the local checkpoint path (config.json +
model.safetensors, src/core/safetensors.zig:32-97), through the C ABI.

Against the oracle's restatement of forecast (pinned by its composition test and quantileLinear's
reference cases), at _ref.reference_bar: twice the reference's own spread between its 8-lane and
16-lane builds on the same forecast (at least 1e-5). Covered: a horizon inside one block (the
chunk forecast itself, bit for bit), several fed-back blocks, a context window that drops its
oldest steps, a last block cut by the horizon, and the end-to-end configuration (Chronos-Bolt-small,
16 series x 512 steps, 2 % NaN) read from a random-init checkpoint written to disk.
"""
import numpy as np
import pytest

import _ref

pytestmark = pytest.mark.gpu

THREADS = 16
LEVELS = np.linspace(0.1, 0.9, 9).astype(np.float32)


def _weights(w):
    a, m = w.arrays, w.meta
    return dict(reg=a["reg"], dec_start=a["dec_start"], rel_table=a["rel_table"], enc=m["enc"], dec=m["dec"],
                enc_final_norm=a["enc_final_norm"], dec_final_norm=a["dec_final_norm"], ie=m["ie"], oe=m["oe"],
                d_model=m["d_model"], heads=w.H, d_ff=m["d_ff"], eps=m["eps"], buckets=m["buckets"],
                max_distance=m["max_distance"])


def _device(w):
    import torch

    cu = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    d = {k: cu(w[k]) for k in ("reg", "dec_start", "rel_table", "enc_final_norm", "dec_final_norm")}
    d["enc"] = [{k: cu(v) for k, v in ly.items()} for ly in w["enc"]]
    d["dec"] = [{k: cu(v) for k, v in ly.items()} for ly in w["dec"]]
    d["ie"], d["oe"] = ({k: cu(v) for k, v in w[b].items()} for b in ("ie", "oe"))
    return d


def _gpu_horizon(ta, w, x, horizon, P, max_ctx, levels=LEVELS):
    import torch

    dv = _device(w)
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    out = torch.full((x.shape[0], horizon, levels.size), -7.0, device="cuda")
    rc = ta.bolt_forecast_horizon(out, xd, horizon, dv["reg"], dv["dec_start"], dv["rel_table"], dv["enc"],
                                  dv["enc_final_norm"], dv["dec"], dv["dec_final_norm"], dv["ie"], dv["oe"],
                                  w["d_model"], w["heads"], w["d_ff"], w["eps"], levels, P, max_ctx)
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _series(seed, b, t_in, nan=0.02):
    rng = np.random.default_rng(seed)
    t = np.arange(t_in)
    x = (10 * np.sin(2 * np.pi * t / 24) + rng.uniform(-0.05, 0.05, (b, 1)) * t +
         rng.standard_normal((b, t_in))).astype(np.float32)
    x[rng.random(x.shape) < nan] = np.nan
    return x


def _small(P=16):
    from tsfm_attn import workloads

    return _weights(workloads.bolt_forward(B=2, n_patch=2, H=2, d_ff=256, n_layers=2, quantiles=9, horizon=P, seed=3))


def test_horizon_inside_one_block_is_the_chunk_forecast(ta, gpu_ready):
    """horizon <= prediction_length: the (b, horizon, q) steps of tsfm_bolt_forecast's (b, q, P)
    output over the last context_length steps, bit for bit."""
    import torch

    P = 16
    w = _small(P)
    x = _series(1, 3, 90)
    got = _gpu_horizon(ta, w, x, 11, P, 64)
    dv = _device(w)
    ctx = torch.from_numpy(np.ascontiguousarray(x[:, -64:])).cuda()
    out = torch.zeros((3, 9 * P), device="cuda")
    rc = ta.bolt_forecast(out, ctx, 64, dv["reg"], dv["dec_start"], dv["rel_table"], dv["enc"], dv["enc_final_norm"],
                          dv["dec"], dv["dec_final_norm"], dv["ie"], dv["oe"], 3, w["d_model"], w["heads"], w["d_ff"],
                          w["eps"])
    assert rc == ta.OK, ta.last_error()
    torch.cuda.synchronize()
    want = out.cpu().numpy().reshape(3, 9, P).transpose(0, 2, 1)[:, :11]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("t_in,max_ctx,horizon", [(70, 96, 50), (130, 64, 33), (200, 2048, 64)])
def test_long_horizon_matches_oracle(ta, orc, orc16, gpu_ready, t_in, max_ctx, horizon):
    P = 16
    w = _small(P)
    x = _series(t_in, 3, t_in)
    got = _gpu_horizon(ta, w, x, horizon, P, max_ctx)
    w8, w16 = (o_.bolt_forecast_horizon(THREADS, x, horizon, w, P, max_ctx, LEVELS) for o_ in (orc, orc16))
    assert np.isfinite(got).all()
    _ref.assert_within_reference_bar(got, w8, w16)


def test_end_to_end_config_from_a_local_checkpoint(ta, orc, orc16, gpu_ready, tmp_path):
    """Chronos-Bolt-small random-init weights written as config.json + model.safetensors, read back
    by tsfm_attn.checkpoint into device tensors; the 16 x 512 sinusoid + trend + noise series with
    2 % NaN: horizon 64 equals the in-memory chunk forecast bit for bit, and horizon 128 (one fed-back
    block over 144 quantile paths) matches the oracle."""
    import torch

    from tsfm_attn import checkpoint, workloads

    wl = workloads.bolt_forward()
    w = _weights(wl)
    cfg = checkpoint.bolt_config_dict(d_model=512, d_ff=2048, num_heads=8, num_layers=6, num_decoder_layers=6,
                                      context_length=2048, patch=16, prediction_length=64, quantiles=LEVELS.tolist())
    checkpoint.write_bolt_checkpoint(str(tmp_path), cfg, w)
    fc = checkpoint.load_bolt(str(tmp_path))
    ctx = np.ascontiguousarray(wl.arrays["ctx"])
    assert ctx.shape == (16, 512) and np.isnan(ctx).mean() > 0.01
    x = torch.from_numpy(ctx).cuda()
    one = fc.forecast(x, 64)
    torch.cuda.synchronize()
    assert np.array_equal(one.cpu().numpy(), _gpu_horizon(ta, w, ctx, 64, 64, 2048))
    two = fc.forecast(x, 128).cpu().numpy()
    assert np.array_equal(two[:, :64], one.cpu().numpy())
    w8, w16 = (o_.bolt_forecast_horizon(THREADS, ctx, 128, w, 64, 2048, LEVELS) for o_ in (orc, orc16))
    _ref.assert_within_reference_bar(two, w8, w16)


def test_horizon_argument_errors(ta, gpu_ready):
    import torch

    w = _small()
    dv = _device(w)
    x = torch.zeros((1, 32), device="cuda")
    out = torch.zeros((1, 8, 9), device="cuda")
    args = (dv["reg"], dv["dec_start"], dv["rel_table"], dv["enc"], dv["enc_final_norm"], dv["dec"],
            dv["dec_final_norm"], dv["ie"], dv["oe"], w["d_model"], w["heads"], w["d_ff"], w["eps"])
    assert ta.bolt_forecast_horizon(out, x, 8, *args, LEVELS[:8], 16, 64) == ta.E_INVALID  # q * P != out width
    assert ta.bolt_forecast_horizon(out, x, 8, *args, np.full(9, 1.5, np.float32), 16, 64) == ta.E_INVALID
    assert ta.bolt_forecast_horizon(out, x, 8, *args, LEVELS, 16, 0) == ta.E_INVALID
    torch.cuda.synchronize()
    assert (out == 0).all()
