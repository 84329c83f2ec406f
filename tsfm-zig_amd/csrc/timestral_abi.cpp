// extern "C" tsfm_timestral_forecast (include/tsfm_attn.h): the Timestral forecaster on the device.
//
// Reference: src/timestral/forecaster.zig forecast (:57-180), forecastRaw (:303-421), blockDecode
// (:423-563), refineBlock (:582-662) and src/timestral/model.zig predictBlock (:220-432), with
// numeric past-only and known-future covariate rows after each series' targets. The forward and
// the mirrored pass of the symmetric average run as one batch: the mirrored series are groups
// batch..2 batch-1 of every launch. With covariates each block's encoder covers its window (the
// context plus the horizon's known futures or blanks), as the reference's does; with known-future
// rows every block re-encodes it.
//
// The reference re-encodes the whole grown context for every decode block (blockDecode calls
// predictBlock on the full context). Without covariates every encoder layer is causal over
// patches (causal time attention, per-slot variate attention, per-token norms and MLP, causal
// per-patch statistics), so the encoder tokens of the context that was already there are the same
// in the next block. With kv_cache set, each time-attention layer keeps its q/k/v rows of every
// encoder token (one (rows, tokens, 3 d) buffer per layer), and a block runs only its new patches
// and its decoder tokens through the layers, their queries attending over the kept keys. Blocks
// that change the prefix run in full: after the context window drops its oldest steps
// (max_context). A group with no observation at all moves its RoPE origin (the first observed
// patch) once the fed-back medians appear; its earlier tokens are invalid keys for every later
// query, so the RoPE tables are recomputed every block and the cache stays exact.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/tsfm_attn.h"
#include "abi_internal.hpp"
#include "launch.hpp"

using tsfm::abi::aligned;
using tsfm::abi::ensure_ready;
using tsfm::abi::fail;
using tsfm::abi::hip_fail;
using tsfm::abi::Plan;

namespace {

constexpr int kActSilu = 1;  // tsfm_resblock.act

// One nn.linear (y = x w^T + bias) with an epilogue, over `rows` packed rows.
hipError_t linear(const float* x, int64_t x_tok, const float* w, int out, int in, const float* bias, float* y,
                  int64_t y_tok, int rows, int epi, const float* resid, hipStream_t s) {
    tsfm::ProjParams p{};
    p.x = x; p.x_tok = x_tok; p.w0 = w; p.w_ld = in; p.alpha = 1.f; p.epi = epi; p.bias = bias;
    p.resid = resid; p.resid_tok = y_tok;
    p.y0 = y; p.y0_tok = y_tok;
    p.tokens = rows; p.seq = rows; p.d_in = in; p.width = out; p.n_out = 1; p.out_dtype = TSFM_DTYPE_F32;
    return tsfm::launch_proj(p, s);
}

// ResBlock(.silu).forward (src/core/resblock.zig:63-79): y = output(silu(hidden(x))) + residual(x),
// biases where given. hbuf: rows x hid, rbuf: rows x out.
hipError_t resblock_silu(const tsfm_resblock& rb, const float* x, int rows, float* y, float* hbuf, float* rbuf,
                         hipStream_t s) {
    hipError_t e = linear(x, rb.in, rb.hidden_w, rb.hid, rb.in, rb.hidden_b, hbuf, rb.hid, rows, tsfm::kEpiSilu,
                          nullptr, s);
    if (e == hipSuccess)
        e = linear(x, rb.in, rb.residual_w, rb.out, rb.in, rb.residual_b, rbuf, rb.out, rows, tsfm::kEpiNone, nullptr,
                   s);
    if (e == hipSuccess)
        e = linear(hbuf, rb.hid, rb.output_w, rb.out, rb.hid, rb.output_b, y, rb.out, rows, tsfm::kEpiResidual, rbuf,
                   s);
    return e;
}

int check_resblock(const tsfm_resblock& rb, int in, int out, bool biases, const char* what) {
    if (rb.act != kActSilu) return fail(TSFM_E_UNSUPPORTED, "%s: activation %d (Timestral uses SiLU, 1)", what, rb.act);
    if (rb.in != in || rb.out != out || rb.hid <= 0)
        return fail(TSFM_E_INVALID, "%s: shape %d -> %d -> %d, expected %d -> . -> %d", what, rb.in, rb.hid, rb.out, in,
                    out);
    if (rb.in % 16 || rb.hid % 16 || rb.out % 4) return fail(TSFM_E_UNSUPPORTED, "%s: widths must be multiples of 16", what);
    if (!rb.hidden_w || !rb.output_w || !rb.residual_w) return fail(TSFM_E_INVALID, "%s: a weight is NULL", what);
    if (biases && (!rb.hidden_b || !rb.output_b || !rb.residual_b)) return fail(TSFM_E_INVALID, "%s: a bias is NULL", what);
    for (const float* p : {rb.hidden_w, rb.output_w, rb.residual_w, rb.hidden_b, rb.output_b, rb.residual_b})
        if (p != nullptr && !aligned(p, 16)) return fail(TSFM_E_UNSUPPORTED, "%s: device pointers must be 16-byte aligned", what);
    return TSFM_OK;
}

}  // namespace

extern "C" int tsfm_timestral_forecast(const tsfm_timestral_forecast_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    const tsfm_timestral_model& M = a->model;
    if (a->flags & ~(TSFM_ATTN_DEVICE_PTRS | TSFM_TIMESTRAL_BF16_ATTN | TSFM_FORECAST_HOST_IO))
        return fail(TSFM_E_INVALID, "unknown flags");
    if (!(a->flags & TSFM_ATTN_DEVICE_PTRS))
        return fail(TSFM_E_UNSUPPORTED, "the Timestral forecast takes device weights (TSFM_ATTN_DEVICE_PTRS; "
                                        "TSFM_FORECAST_HOST_IO for host inputs and outputs)");
    if (a->batch < 0 || a->variates <= 0 || a->len <= 0 || a->horizon <= 0)
        return fail(TSFM_E_INVALID, "bad batch, variates, len or horizon");
    if (a->batch == 0) return TSFM_OK;
    const int ps = M.patch, d = M.d_model, nh = M.heads, hid = M.mlp_hidden, q = M.n_quantiles;
    if (M.head_dim != 64) return fail(TSFM_E_UNSUPPORTED, "head_dim %d (supported: 64)", M.head_dim);
    if (ps <= 0 || ps > 256 || d != nh * 64 || hid <= 0 || hid % 16 || d % 16)
        return fail(TSFM_E_UNSUPPORTED, "patch %d, d_model %d, heads %d, mlp_hidden %d", ps, d, nh, hid);
    if (q < 1 || q > 32 || M.quantile_knots == nullptr) return fail(TSFM_E_UNSUPPORTED, "1 to 32 quantile knots");
    if (M.rope_dim <= 0 || M.rope_dim % 2 || M.rope_dim > 64) return fail(TSFM_E_INVALID, "bad rope_dim %d", M.rope_dim);
    if (a->n_past < 0 || a->n_known < 0) return fail(TSFM_E_INVALID, "negative covariate count");
    if ((a->n_past > 0 && !a->past) || (a->n_known > 0 && !a->known))
        return fail(TSFM_E_INVALID, "a covariate count without its array");
    // forecaster.zig:104: covariates given but no rows (error.InvalidInput)
    if ((a->past && a->n_past == 0) || (a->known && a->n_known == 0))
        return fail(TSFM_E_INVALID, "a covariate array with no rows (error.InvalidInput)");
    if ((a->past || a->known) && !M.covariate_enabled)
        return fail(TSFM_E_UNSUPPORTED, "covariates with covariate_enabled off (error.CovariatesUnsupported)");
    if ((int64_t)a->variates + a->n_past + a->n_known > TSFM_VARIATE_MAX_ROWS)
        return fail(TSFM_E_UNSUPPORTED, "at most %d rows (variates and covariates) per series", TSFM_VARIATE_MAX_ROWS);
    if ((a->flags & TSFM_TIMESTRAL_BF16_ATTN) && M.use_asinh)
        return fail(TSFM_E_UNSUPPORTED, "bf16 time attention with use_asinh: the sinh expansion of the head "
                                        "outputs takes the bf16 rounding past the half-precision bar");
    if (M.block_size <= 0 || M.n_layers < 0 || (M.n_layers > 0 && M.layers == nullptr))
        return fail(TSFM_E_INVALID, "bad block_size or layers");
    if (!a->inputs || !a->observed || !a->out || !M.forecast_query || !M.out_norm)
        return fail(TSFM_E_INVALID, "inputs, observed, out, forecast_query and out_norm are required");
    if (!aligned(M.forecast_query, 16) || !aligned(M.out_norm, 16))
        return fail(TSFM_E_UNSUPPORTED, "device pointers must be 16-byte aligned");
    int median = -1;
    for (int i = 0; i < q; i++) {
        if (i > 0 && !(M.quantile_knots[i - 1] < M.quantile_knots[i]))
            return fail(TSFM_E_INVALID, "quantile knots must increase");
        if (M.quantile_knots[i] == 0.5) median = i;
    }
    if (median < 0) return fail(TSFM_E_INVALID, "the quantile knots need 0.5");
    if (a->symmetric_averaging)
        for (int i = 0; i < q; i++)
            if (std::fabs(M.quantile_knots[i] + M.quantile_knots[q - 1 - i] - 1.0) > 1e-9)
                return fail(TSFM_E_INVALID, "symmetric averaging needs symmetric quantile levels");
    int rc;
    if ((rc = check_resblock(M.patch_proj, 2 * ps, d, true, "patch_proj")) != TSFM_OK) return rc;
    if ((rc = check_resblock(M.head, d, ps * q, false, "head")) != TSFM_OK) return rc;
    int n_time = 0;
    for (int li = 0; li < M.n_layers; li++) {
        const tsfm_timestral_layer& ly = M.layers[li];
        if (ly.n_attn < 1 || ly.n_attn > 2) return fail(TSFM_E_INVALID, "layer %d: n_attn %d", li, ly.n_attn);
        for (int ai = 0; ai < ly.n_attn; ai++) {
            const tsfm_timestral_attn& at = ly.attn[ai];
            if (!at.norm || !at.qkv || !at.out) return fail(TSFM_E_INVALID, "layer %d: a weight is NULL", li);
            for (const float* p : {at.norm, at.qkv, at.out, at.gate})
                if (p != nullptr && !aligned(p, 16))
                    return fail(TSFM_E_UNSUPPORTED, "device pointers must be 16-byte aligned");
            n_time += at.is_time ? 1 : 0;
        }
        if (!ly.mlp_norm || !ly.w12 || !ly.w3) return fail(TSFM_E_INVALID, "layer %d: an MLP weight is NULL", li);
        for (const float* p : {ly.mlp_norm, ly.w12, ly.w3})
            if (!aligned(p, 16)) return fail(TSFM_E_UNSUPPORTED, "device pointers must be 16-byte aligned");
    }
    if (a->n_known > 0) {
        // Config.supportsKnownCovariates (src/timestral/config.zig:49-70): some time op must be
        // followed by at least one more time op and at least one variate op.
        std::vector<bool> ops;
        for (int li = 0; li < M.n_layers; li++)
            for (int ai = 0; ai < M.layers[li].n_attn; ai++) ops.push_back(M.layers[li].attn[ai].is_time != 0);
        bool routes = false;
        for (size_t i = 0; i < ops.size() && !routes; i++) {
            if (!ops[i]) continue;
            bool any_time = false, any_variate = false;
            for (size_t j = i + 1; j < ops.size(); j++) {
                any_time = any_time || ops[j];
                any_variate = any_variate || !ops[j];
            }
            routes = any_time && any_variate;
        }
        if (!routes)
            return fail(TSFM_E_UNSUPPORTED, "known covariates: the layer schedule cannot route them to the targets "
                                            "(error.KnownCovariatesUnsupported)");
    }
    if (a->flags & TSFM_FORECAST_HOST_IO) {
        tsfm_timestral_forecast_args dv = *a;
        dv.flags &= ~TSFM_FORECAST_HOST_IO;
        const size_t rows = (size_t)a->batch * a->variates, L = (size_t)a->len, H = (size_t)a->horizon;
        return tsfm::abi::run_host_io(
            {{a->inputs, rows * L * 4, reinterpret_cast<const void**>(&dv.inputs)},
             {a->observed, rows * L, reinterpret_cast<const void**>(&dv.observed)},
             {a->past, (size_t)a->batch * a->n_past * L * 4, reinterpret_cast<const void**>(&dv.past)},
             {a->known, (size_t)a->batch * a->n_known * (L + H) * 4, reinterpret_cast<const void**>(&dv.known)}},
            {{a->out, rows * H * q * 4, const_cast<const void**>(reinterpret_cast<void**>(&dv.out))}},
            [&](hipStream_t s) {
                dv.stream = s;
                return tsfm_timestral_forecast(&dv);
            });
    }
    if ((rc = ensure_ready()) != TSFM_OK) return rc;

    // ---- sizes ----
    const int V = a->variates, R = a->batch * V, n_cov = a->n_past + a->n_known, vall = V + n_cov;
    const bool cov = n_cov > 0;
    const int groups = a->symmetric_averaging ? 2 * a->batch : a->batch, rows = groups * vall;
    uint32_t role_words[TSFM_VARIATE_MAX_ROWS / 4] = {};  // model.Role per row of a series, byte i = row i
    for (int i = 0; i < vall; i++)
        role_words[i / 4] |= (uint32_t)(i < V ? 0 : i < V + a->n_past ? 1 : tsfm::kRoleKnown) << (8 * (i % 4));
    const int max_context = a->max_context > 0 ? a->max_context : M.context_length;
    if (max_context <= 0) return fail(TSFM_E_INVALID, "max_context");
    const int per_shot = std::min(a->per_shot_patches > 0 ? a->per_shot_patches : 32, M.block_size);
    const int keep = std::min(a->len, max_context), t_first = (keep + ps - 1) / ps * ps;
    const int total_patches = (a->horizon + ps - 1) / ps;
    const int cap_t = t_first + total_patches * ps, cap_p = cap_t / ps;
    const int cap_tok = cap_p + per_shot + (cov ? per_shot : 0), sl_max = cap_tok;  // cov: window + decoder
    const int hpad = total_patches * ps;
    if ((int64_t)rows * cap_tok * 3 * d > 0x7fffffffLL * 4) return fail(TSFM_E_UNSUPPORTED, "too large");
    hipStream_t s = static_cast<hipStream_t>(a->stream);

    Plan plan;
    const size_t R4 = (size_t)rows * 4;
    const size_t at_ctx0 = plan.take((size_t)rows * cap_t * 4), at_ctx1 = plan.take((size_t)rows * cap_t * 4);
    const size_t at_mk0 = plan.take((size_t)rows * cap_t), at_mk1 = plan.take((size_t)rows * cap_t);
    const size_t at_loc = plan.take(R4 * cap_p), at_scale = plan.take(R4 * cap_p), at_kv = plan.take((size_t)rows * cap_p);
    const size_t at_state = plan.take((size_t)rows * 4 * 8), at_fold = plan.take((size_t)rows * 3 * 8);
    const size_t at_rfirst = plan.take(R4), at_first = plan.take((size_t)groups * 4), at_nonneg = plan.take((size_t)R);
    const size_t at_bounds = plan.take(R4 * 2);  // per context row
    const size_t tab = (size_t)groups * cap_tok * 32 * 4;
    const size_t at_cos = plan.take(tab), at_sin = plan.take(tab);
    const size_t at_feats = plan.take(R4 * cap_p * 2 * ps), at_eh = plan.take(R4 * cap_p * M.patch_proj.hid);
    const size_t at_er = plan.take(R4 * cap_p * d), at_emb = plan.take(R4 * cap_p * d);
    const size_t act = R4 * sl_max * d;
    const size_t at_x = plan.take(act), at_xn = plan.take(act), at_oa = plan.take(act), at_g = plan.take(act);
    const size_t at_vq = plan.take(act * 3), at_h = plan.take(R4 * sl_max * 2 * hid), at_a = plan.take(R4 * sl_max * hid);
    std::vector<size_t> at_cache((size_t)n_time);
    for (int i = 0; i < n_time; i++) at_cache[(size_t)i] = plan.take(R4 * cap_tok * 3 * d);
    const size_t at_dec = plan.take(R4 * per_shot * d), at_hh = plan.take(R4 * per_shot * M.head.hid);
    const size_t at_hr = plan.take(R4 * per_shot * ps * q), at_raw = plan.take(R4 * per_shot * ps * q);
    const size_t at_qs = plan.take(R4 * per_shot * ps * q), at_fr = plan.take(R4 * per_shot * 2);
    const size_t at_mir = plan.take((size_t)R * a->horizon * q * 4);
    const size_t at_part = plan.take(tsfm::kSplitWorkspaceBytes);
    const size_t planes_n = tsfm::proj_plane_bytes((int64_t)rows * sl_max, std::max(d, hid), std::max(3 * d, 2 * hid));
    const size_t at_planes = plan.take(planes_n);
    const size_t at_kf = plan.take((size_t)rows * hpad * 4 + 4), at_kfm = plan.take((size_t)rows * hpad + 1);
    const size_t at_noasinh = plan.take((size_t)rows);
    char* buf = nullptr;
    bool owned = false;
    hipError_t e = tsfm::abi::scratch_acquire(s, tsfm::abi::kSlotTimestralForecast, plan.off, &buf, &owned);
    if (e != hipSuccess) return hip_fail(e, "forecast scratch allocation");
    auto F = [&](size_t at) { return reinterpret_cast<float*>(buf + at); };
    auto U8 = [&](size_t at) { return reinterpret_cast<uint8_t*>(buf + at); };
    tsfm::SplitWorkspace ws(F(at_part));
    tsfm::PlaneWorkspace pws(buf + at_planes, planes_n);

    float* ctx[2] = {F(at_ctx0), F(at_ctx1)};
    uint8_t* mask[2] = {U8(at_mk0), U8(at_mk1)};
    int cur = 0;
    float *loc = F(at_loc), *scale = F(at_scale);
    uint8_t* kv = U8(at_kv);
    double* state = reinterpret_cast<double*>(buf + at_state);
    double* fold = reinterpret_cast<double*>(buf + at_fold);
    int* row_first = reinterpret_cast<int*>(buf + at_rfirst);
    int* first_obs = reinterpret_cast<int*>(buf + at_first);
    float *cos_t = F(at_cos), *sin_t = F(at_sin);
    float *X = F(at_x), *XN = F(at_xn), *OA = F(at_oa), *G = F(at_g), *VQ = F(at_vq), *H = F(at_h), *A = F(at_a);
    float* qs = F(at_qs);

    tsfm::TsRope rope{};
    for (int i = 0; i < M.rope_dim / 2; i++)
        rope.inv_freq[i] = 1.0f / std::pow(M.rope_theta, (float)(2 * i) / (float)M.rope_dim);
    tsfm::TsHead hp{};
    hp.ps = ps; hp.q = q; hp.median = median; hp.use_asinh = M.use_asinh ? 1 : 0; hp.wf = M.quantile_width_factor;
    for (int i = median + 1; i < q; i++) hp.widths[i] = (float)(M.quantile_knots[i] - M.quantile_knots[i - 1]);
    for (int i = 0; i < median; i++) hp.widths[i] = (float)(M.quantile_knots[i + 1] - M.quantile_knots[i]);
    const float sm_scale = 1.0f / std::sqrt(64.0f);
    // bf16 time attention: the layer caches hold bf16 q/k/v (the same buffers, half used), and the
    // attention output goes to VQ as bf16 (VQ serves only the variate layers otherwise).
    const bool half = (a->flags & TSFM_TIMESTRAL_BF16_ATTN) != 0;
    uint16_t* OH = reinterpret_cast<uint16_t*>(VQ);

    float* const out = a->out;
    const float cap_k = a->quantile_real_cap_k;
    const float eps = M.norm_eps;

    auto run = [&]() -> hipError_t {
        tsfm::TsContextParams cp{};
        cp.inputs = a->inputs; cp.observed = a->observed; cp.past = a->past; cp.known = a->known;
        cp.batch = a->batch; cp.V = V; cp.n_past = a->n_past; cp.n_known = a->n_known; cp.vall = vall; cp.rows = rows;
        cp.t0 = a->len; cp.keep = keep; cp.t = t_first; cp.horizon = a->horizon; cp.hpad = hpad; cp.cap_t = cap_t;
        cp.ctx = ctx[0]; cp.mask = mask[0]; cp.kf = F(at_kf); cp.kfm = U8(at_kfm); cp.nonneg = U8(at_nonneg);
        hipError_t e2 = tsfm::launch_ts_context(cp, s);
        if (e2 != hipSuccess) return e2;
        // Known-future rows attend over the whole window and take whole-window statistics: every
        // token changes when the window grows. Past-only rows are causal like the targets; their
        // blank future patches (read by no context token or decoder query) leave the carried
        // statistics unchanged (zero weight) and are recomputed as context in the next block.
        const bool cache = a->kv_cache != 0 && a->n_known == 0;
        const int known_from = V + a->n_past;  // first known-future row of a series
        int t = t_first, remaining = total_patches, done = 0;
        int stats_from = 0;  // first step of the window whose statistics are not computed yet
        int p0 = 0;          // first token of this block's encoder run: the cache holds tokens [0, p0)
        for (int block_no = 0; remaining > 0; block_no++) {
            const int h = std::min(per_shot, remaining), blen = h * ps, l = t / ps;
            // With covariates the encoder covers the window [0, t + blen): the block's known
            // futures and blanks are written after the context first (model.zig:253-273).
            const int ne = cov ? l + h : l, m = ne - p0, sl = m + h, w = ne * ps;
            if (cov && (e2 = tsfm::launch_ts_window(ctx[cur], mask[cur], cap_t, t, blen, F(at_kf), U8(at_kfm), hpad,
                                                    done, vall, known_from, rows, s)) != hipSuccess)
                return e2;
            // 1. causal statistics, key validity and first observation of the new steps
            tsfm::TsStatsParams sp{};
            sp.ctx = ctx[cur]; sp.mask = mask[cur]; sp.cap_t = cap_t; sp.cap_p = cap_p; sp.rows = rows; sp.ps = ps;
            sp.from = stats_from; sp.t = w; sp.attend_missing = M.attend_missing ? 1 : 0; sp.min_scale = M.minimum_scale;
            sp.loc = loc; sp.scale = scale; sp.key_valid = kv; sp.row_first = row_first; sp.state = state; sp.fold = fold;
            if ((e2 = tsfm::launch_ts_stats(sp, s)) != hipSuccess) return e2;
            if (a->n_known > 0 &&
                (e2 = tsfm::launch_ts_known_stats(ctx[cur], mask[cur], cap_t, w, ps, rows, vall, known_from,
                                                  M.minimum_scale, loc, scale, cap_p, U8(at_noasinh), s)) != hipSuccess)
                return e2;
            if (block_no == 0 && cap_k > 0 &&
                (e2 = tsfm::launch_ts_cap_bounds(ctx[cur], mask[cur], cap_t, t, ps, scale, cap_p, rows, cap_k,
                                                 F(at_bounds), s)) != hipSuccess)
                return e2;
            // The RoPE tables follow each group's first observed patch, recomputed every block: a
            // group with no observation gets its origin from the first fed-back medians. Its earlier
            // tokens are then invalid keys for every later query (no observed patch before them), so
            // their cached K/V, RoPE'd at the old origin, carry zero weight, and the new tokens are
            // RoPE'd at the new origin exactly as a re-encoding would: the cache stays exact without
            // the host learning which groups had no observation.
            if ((e2 = tsfm::launch_ts_rope_tables(row_first, groups, vall, cap_tok, ne, ne - l, rope, cos_t, sin_t,
                                                  first_obs, s)) != hipSuccess)
                return e2;
            // 2. patch embedding of the new patches; [encoder tokens; forecast queries]
            if ((e2 = tsfm::launch_ts_features(ctx[cur], mask[cur], cap_t, loc, scale, cap_p, rows, p0, ne, ps,
                                               M.use_asinh ? 1 : 0, a->n_known > 0 ? U8(at_noasinh) : nullptr,
                                               F(at_feats), s)) != hipSuccess ||
                (e2 = resblock_silu(M.patch_proj, F(at_feats), rows * m, F(at_emb), F(at_eh), F(at_er), s)) !=
                    hipSuccess ||
                (e2 = tsfm::launch_ts_assemble(F(at_emb), M.forecast_query, X, rows, m, h, d, s)) != hipSuccess)
                return e2;
            // 3. the layers (runTransformer, model.zig:465-481)
            const int toks = rows * sl;
            int ti = 0;
            for (int li = 0; li < M.n_layers; li++) {
                const tsfm_timestral_layer& ly = M.layers[li];
                for (int ai = 0; ai < ly.n_attn; ai++) {
                    const tsfm_timestral_attn& at = ly.attn[ai];
                    if ((e2 = tsfm::launch_rms_norm(X, d, XN, d, at.norm, toks, d, eps, s)) != hipSuccess) return e2;
                    tsfm::ProjParams pp{};
                    pp.x = XN; pp.x_tok = d; pp.w_ld = d; pp.alpha = 1.f; pp.epi = tsfm::kEpiNone;
                    pp.w0 = at.qkv; pp.w1 = at.qkv + (int64_t)d * d; pp.w2 = at.qkv + 2 * (int64_t)d * d; pp.w3 = at.gate;
                    pp.tokens = toks; pp.seq = sl; pp.d_in = d; pp.width = d; pp.n_out = at.gate ? 4 : 3;
                    pp.out_dtype = TSFM_DTYPE_F32;
                    pp.y3 = G; pp.y3_tok = d;
                    if (at.is_time) {
                        // q/k/v of the block's tokens into the layer's cache at token p0, RoPE'd with
                        // the rows p0.. of each group's table (timeAttention :493-513).
                        float* T = F(at_cache[(size_t)ti++]);
                        uint16_t* Th = reinterpret_cast<uint16_t*>(T);
                        auto el = [&](int64_t e) -> void* { return half ? (void*)(Th + e) : (void*)(T + e); };
                        const int64_t tb = (int64_t)cap_tok * 3 * d;
                        pp.y0 = el((int64_t)p0 * 3 * d); pp.y1 = el((int64_t)p0 * 3 * d + d);
                        pp.y2 = el((int64_t)p0 * 3 * d + 2 * d);
                        if (half) {  // q/k/v rounded to bf16; the gate stays f32 (its own product)
                            pp.out_dtype = TSFM_DTYPE_BF16; pp.n_out = 3; pp.w3 = nullptr; pp.y3 = nullptr;
                        }
                        pp.y0_tok = pp.y1_tok = pp.y2_tok = 3 * d;
                        pp.y0_batch = pp.y1_batch = pp.y2_batch = tb;
                        pp.rope_cos = cos_t + (int64_t)p0 * 32; pp.rope_sin = sin_t + (int64_t)p0 * 32;
                        pp.rope_table_stride = (int64_t)cap_tok * 32; pp.rope_rows_per_table = vall; pp.rope_row0 = 0;
                        if ((e2 = tsfm::launch_proj(pp, s)) != hipSuccess) return e2;
                        if (half && at.gate &&
                            (e2 = linear(XN, d, at.gate, d, d, nullptr, G, d, toks, tsfm::kEpiNone, nullptr, s)) !=
                                hipSuccess)
                            return e2;
                        auto attend = [&](const tsfm::Params& q, int msk) {
                            return half ? tsfm::launch_attn_half(q, true, msk, tsfm::BIAS_NONE, false, s)
                                        : tsfm::launch_attn_f32(q, msk, tsfm::BIAS_NONE, false, s);
                        };
                        // TimeJob.attend (:580-635): encoder queries causal over the valid keys, then
                        // the decoder queries over the valid context keys and their own chain.
                        tsfm::Params ap{};
                        ap.q = el((int64_t)p0 * 3 * d); ap.k = el(d); ap.v = el(2 * d);
                        ap.o = half ? (void*)OH : (void*)OA;
                        ap.q_tok = ap.k_tok = ap.v_tok = 3 * d; ap.q_batch = ap.k_batch = ap.v_batch = tb;
                        ap.o_tok = d; ap.o_batch = (int64_t)sl * d;
                        ap.key_valid = kv; ap.kv_batch = cap_p;
                        ap.B = rows; ap.H = nh; ap.n_q = m; ap.n_k = ne; ap.q_pos0 = p0; ap.scale = sm_scale;
                        if (!cov) {
                            if ((e2 = attend(ap, TSFM_MASK_CAUSAL_KEYS)) != hipSuccess) return e2;
                        } else {
                            // Known-future rows read every valid key (TimeJob.attend :600-609): one launch
                            // per row of a series, its groups batched, with that row's mask.
                            for (int i = 0; i < vall; i++) {
                                tsfm::Params ri = ap;
                                const int64_t esz = half ? 2 : 4;
                                ri.q = (char*)ap.q + i * tb * esz; ri.k = (char*)ap.k + i * tb * esz;
                                ri.v = (char*)ap.v + i * tb * esz;
                                ri.o = (char*)ap.o + i * (int64_t)sl * d * (half ? 2 : 4);
                                ri.q_batch = ri.k_batch = ri.v_batch = vall * tb; ri.o_batch = vall * (int64_t)sl * d;
                                ri.key_valid = kv + (int64_t)i * cap_p; ri.kv_batch = (int64_t)vall * cap_p;
                                ri.B = groups;
                                if ((e2 = attend(ri, i >= known_from ? TSFM_MASK_FULL_KEYS : TSFM_MASK_CAUSAL_KEYS)) !=
                                    hipSuccess)
                                    return e2;
                            }
                        }
                        // Decoder queries read the valid context keys [0, l) and their own chain from ne.
                        ap.q = el((int64_t)ne * 3 * d);
                        ap.o = half ? (void*)(OH + (int64_t)m * d) : (void*)(OA + (int64_t)m * d);
                        ap.n_q = h; ap.n_k = ne + h; ap.q_pos0 = ne; ap.ctx_keys = l; ap.chain_start = ne;
                        if ((e2 = attend(ap, TSFM_MASK_DECODER)) != hipSuccess) return e2;
                        if (half) {
                            if ((e2 = tsfm::launch_ts_from_bf16(OH, at.gate ? G : nullptr, OA, (int64_t)toks * d, s)) !=
                                hipSuccess)
                                return e2;
                        } else if (at.gate && (e2 = tsfm::launch_ts_mul_sigmoid(OA, G, (int64_t)toks * d, s)) != hipSuccess) {
                            return e2;
                        }
                    } else {
                        // variateAttention (:525-544): the block's token slots only, gate fused.
                        pp.y0 = VQ; pp.y1 = VQ + d; pp.y2 = VQ + 2 * d;
                        pp.y0_tok = pp.y1_tok = pp.y2_tok = 3 * d;
                        if ((e2 = tsfm::launch_proj(pp, s)) != hipSuccess) return e2;
                        tsfm::VariateParams vp{};
                        vp.qkv = VQ; vp.qkv_row = (int64_t)sl * 3 * d; vp.qkv_tok = 3 * d;
                        vp.o = OA; vp.o_row = (int64_t)sl * d; vp.o_tok = d;
                        vp.gate = at.gate ? G : nullptr; vp.gate_row = (int64_t)sl * d; vp.gate_tok = d;
                        vp.key_valid = kv + p0; vp.kv_row = cap_p;
                        vp.groups = groups; vp.vall = vall; vp.n_tok = sl; vp.n_enc = m; vp.heads = nh; vp.cov = cov ? 1 : 0;
                        for (int i = 0; i < TSFM_VARIATE_MAX_ROWS / 4; i++) vp.roles[i] = role_words[i];
                        vp.scale = sm_scale;
                        if ((e2 = tsfm::launch_variate(vp, s)) != hipSuccess) return e2;
                    }
                    if ((e2 = linear(OA, d, at.out, d, d, nullptr, X, d, toks, tsfm::kEpiResidual, X, s)) != hipSuccess)
                        return e2;
                }
                if ((e2 = tsfm::launch_rms_norm(X, d, XN, d, ly.mlp_norm, toks, d, eps, s)) != hipSuccess ||
                    (e2 = linear(XN, d, ly.w12, 2 * hid, d, nullptr, H, 2 * hid, toks, tsfm::kEpiNone, nullptr, s)) !=
                        hipSuccess ||
                    (e2 = tsfm::launch_ts_mul_silu(H, A, toks, hid, s)) != hipSuccess ||
                    (e2 = linear(A, hid, ly.w3, d, hid, nullptr, X, d, toks, tsfm::kEpiResidual, X, s)) != hipSuccess)
                    return e2;
            }
            // 4. the head on the decoder tokens, the monotone quantiles, refineBlock
            float* dec = F(at_dec);
            if ((e2 = hipMemcpy2DAsync(dec, (size_t)h * d * 4, X + (int64_t)m * d, (size_t)sl * d * 4,
                                       (size_t)h * d * 4, (size_t)rows, hipMemcpyDeviceToDevice, s)) != hipSuccess ||
                (e2 = tsfm::launch_rms_norm(dec, d, dec, d, M.out_norm, rows * h, d, eps, s)) != hipSuccess ||
                (e2 = resblock_silu(M.head, dec, rows * h, F(at_raw), F(at_hh), F(at_hr), s)) != hipSuccess ||
                (e2 = tsfm::launch_ts_head_finish(F(at_raw), loc, scale, cap_p, l, rows, h, hp, qs, s)) != hipSuccess)
                return e2;
            if (h > 1 && (e2 = tsfm::launch_ts_refine(qs, loc, scale, cap_p, l, fold, rows, h, ps, q, median,
                                                      M.minimum_scale, F(at_fr), s)) != hipSuccess)
                return e2;
            if ((e2 = tsfm::launch_ts_store_block(qs, rows, a->batch, vall, V, blen, done, a->horizon, q, out, F(at_mir),
                                                  s)) != hipSuccess)
                return e2;
            remaining -= h;
            done += blen;
            if (remaining == 0) break;
            // 5. the medians become context (blockDecode :512-560)
            if ((e2 = tsfm::launch_ts_feedback(qs, rows, vall, V, blen, q, median, a->extreme_value_threshold,
                                               ctx[cur], mask[cur], cap_t, t, s)) != hipSuccess)
                return e2;
            const int nt = t + blen;
            if (nt > max_context) {
                const int keep_t = std::max(ps, max_context / ps * ps);
                if ((e2 = tsfm::launch_ts_slide(ctx[cur], mask[cur], ctx[1 - cur], mask[1 - cur], rows, cap_t,
                                                nt - keep_t, keep_t, s)) != hipSuccess)
                    return e2;
                cur = 1 - cur;
                t = keep_t;
                stats_from = 0;
                p0 = 0;
            } else if (cache) {
                stats_from = t;
                p0 = l;
                t = nt;
            } else {
                stats_from = 0;  // re-encode the grown context, as the reference does
                p0 = 0;
                t = nt;
            }
        }
        return tsfm::launch_ts_final(out, F(at_mir), F(at_bounds), U8(at_nonneg), R, V, vall, a->horizon, q,
                                     cap_k > 0 ? 1 : 0,
                                     a->symmetric_averaging ? 1 : 0, a->clip_nonnegative ? 1 : 0, s);
    };
    e = run();
    const hipError_t f = owned ? hipFreeAsync(buf, s) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "Timestral forecast launch");
    if (f != hipSuccess) return hip_fail(f, "forecast scratch release");
    return TSFM_OK;
}
