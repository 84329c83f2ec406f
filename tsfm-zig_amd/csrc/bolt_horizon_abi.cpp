// extern "C" tsfm_bolt_forecast_horizon (include/tsfm_attn.h): Chronos-Bolt forecaster.forecast
// (src/chronos_bolt/forecaster.zig:22-78) on the device, any horizon.
//
// Block 0 is tsfm_bolt_forecast over the last context_length steps of each series. Later blocks
// run the model over batch * q rows, one per quantile path (window kept on the device, two
// buffers used in turn), and reduce each series' q * q outputs per step to q empirical quantiles.
// Everything is queued on the caller's stream; nothing is synchronised.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/tsfm_attn.h"
#include "abi_internal.hpp"
#include "launch.hpp"

using tsfm::abi::aligned;
using tsfm::abi::ensure_ready;
using tsfm::abi::fail;
using tsfm::abi::hip_fail;
using tsfm::abi::Plan;

extern "C" int tsfm_bolt_forecast_horizon(const tsfm_bolt_horizon_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (!(a->model.flags & TSFM_ATTN_DEVICE_PTRS))
        return fail(TSFM_E_UNSUPPORTED, "the forecast takes device weights (TSFM_ATTN_DEVICE_PTRS; TSFM_FORECAST_HOST_IO "
                                        "for host inputs and outputs)");
    const int64_t b = a->model.batch;
    const int q = a->n_quantiles, P = a->prediction_length, ps = a->patch;
    if (b < 0 || a->t_in <= 0 || a->horizon <= 0 || ps <= 0 || P <= 0 || a->context_length <= 0)
        return fail(TSFM_E_INVALID, "bad batch, t_in, horizon, patch, prediction_length or context_length");
    if (q < 1 || q > 16 || a->quantile_levels == nullptr) return fail(TSFM_E_UNSUPPORTED, "1 to 16 quantile levels");
    if (a->model.output_embed.out != q * P) return fail(TSFM_E_INVALID, "output_embed.out must be n_quantiles * P");
    if (a->inputs == nullptr || a->out == nullptr) return fail(TSFM_E_INVALID, "inputs and out are required");
    if (b == 0) return TSFM_OK;
    if (b * q > 0x7fffffff / std::max(a->context_length, q * P))
        return fail(TSFM_E_UNSUPPORTED, "batch * quantiles * context too large");
    if (a->model.flags & TSFM_FORECAST_HOST_IO) {
        tsfm_bolt_horizon_args d = *a;
        d.model.flags &= ~TSFM_FORECAST_HOST_IO;
        return tsfm::abi::run_host_io(
            {{a->inputs, (size_t)(b * a->t_in) * 4, reinterpret_cast<const void**>(&d.inputs)}},
            {{a->out, (size_t)(b * a->horizon * q) * 4, const_cast<const void**>(reinterpret_cast<void**>(&d.out))}},
            [&](hipStream_t s) {
                d.model.stream = s;
                return tsfm_bolt_forecast_horizon(&d);
            });
    }
    tsfm::BoltLevels lv{};
    for (int i = 0; i < q; i++) {
        lv.v[i] = a->quantile_levels[i];
        if (!(lv.v[i] >= 0.f && lv.v[i] <= 1.f)) return fail(TSFM_E_INVALID, "quantile levels must be in [0, 1]");
    }
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(a->model.stream);
    const int len0 = std::min(a->t_in, a->context_length);
    const bool more = a->horizon > P;
    const int64_t rows = b * q;
    Plan plan;
    const size_t pred_at = plan.take((size_t)(rows * P) * 4);
    const size_t cur_at0 = plan.take(more ? (size_t)rows * a->context_length * 4 : 0);
    const size_t cur_at1 = plan.take(more ? (size_t)rows * a->context_length * 4 : 0);
    const size_t raw_at = plan.take(more ? (size_t)(rows * q * P) * 4 : 0);
    char* buf = nullptr;
    bool owned = false;
    hipError_t e = tsfm::abi::scratch_acquire(s, tsfm::abi::kSlotBoltHorizon, plan.off, &buf, &owned);
    if (e != hipSuccess) return hip_fail(e, "forecast scratch allocation");
    float* pred = reinterpret_cast<float*>(buf + pred_at);
    float* cur[2] = {reinterpret_cast<float*>(buf + cur_at0), reinterpret_cast<float*>(buf + cur_at1)};
    float* raw = reinterpret_cast<float*>(buf + raw_at);

    auto block = [&](const float* ctx, int64_t stride, int64_t offset, int len, int64_t n, float* dst) {
        tsfm_bolt_forecast_args f{};
        f.model = a->model;
        f.model.batch = (int32_t)n;
        f.model.n_patch = (len + ps - 1) / ps;
        f.ctx = ctx; f.stride = stride; f.offset = offset; f.len = len; f.patch = ps; f.norm_eps = a->norm_eps;
        f.out = dst;
        return tsfm_bolt_forecast(&f);
    };
    rc = block(a->inputs, a->t_in, a->t_in - len0, len0, b, pred);
    if (rc == TSFM_OK) {
        e = tsfm::launch_bolt_store_block(pred, (int)b, q, P, a->horizon, 0, a->out, s);
        int done = std::min(P, a->horizon), len = len0, which = 0;
        bool first = true;
        while (e == hipSuccess && rc == TSFM_OK && done < a->horizon) {
            const int new_len = std::min(len + P, a->context_length);
            // Row (s, qi) of the first window is series s's context; later ones the previous window.
            e = first ? tsfm::launch_bolt_window(a->inputs, a->t_in, a->t_in - len0, len, q, pred, P, cur[which], new_len,
                                                 (int)rows, s)
                      : tsfm::launch_bolt_window(cur[which ^ 1], len, 0, len, 1, pred, P, cur[which], new_len, (int)rows,
                                                 s);
            if (e != hipSuccess) break;
            first = false;
            len = new_len;
            if ((rc = block(cur[which], len, 0, len, rows, raw)) != TSFM_OK) break;
            if ((e = tsfm::launch_bolt_sample_quantiles(raw, (int)b, q, P, lv, pred, s)) != hipSuccess ||
                (e = tsfm::launch_bolt_store_block(pred, (int)b, q, P, a->horizon, done, a->out, s)) != hipSuccess)
                break;
            done += P;
            which ^= 1;
        }
    }
    const hipError_t f = owned ? hipFreeAsync(buf, s) : hipSuccess;
    if (rc != TSFM_OK) return rc;
    if (e != hipSuccess) return hip_fail(e, "forecast launch");
    if (f != hipSuccess) return hip_fail(f, "forecast scratch release");
    return TSFM_OK;
}
