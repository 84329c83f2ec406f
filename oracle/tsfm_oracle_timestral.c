/*
 * tsfm_oracle_timestral.c -- CPU oracle: the Timestral model forward and forecaster.
 *
 * TEST INFRASTRUCTURE ONLY (see tsfm_oracle.h): what the device Timestral path is checked against, never
 * linked or called by the product.
 *
 * Restates, for series whose rows are all target variates (no covariates):
 *   Model.patchStats / StatsJob        src/timestral/model.zig:210-216, 712-750
 *   Model.predictBlock                 src/timestral/model.zig:220-432 (cov = false)
 *   Model.runTransformer               src/timestral/model.zig:434-482
 *   Model.timeAttention / variate      src/timestral/model.zig:487-544
 *   ResBlock(.silu).forward            src/core/resblock.zig:63-79
 *   nn.siluInPlace / mulSilu / softplus / clampNonfinite   src/core/nn.zig:399-420, 516-563
 *   forecaster forecastRaw / blockDecode / refineBlock / forecast / finish
 *                                      src/timestral/forecaster.zig:57-180, 303-421, 423-563, 565-662
 *   encodingTarget / encodeCategorical / targetEncode / slotOf
 *                                      src/timestral/forecaster.zig:201-301
 * with the same arithmetic as the Zig (f32 unfused, f64 where the reference uses f64).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "tsfm_oracle.h"

#ifndef ORC_LANES
#define ORC_LANES 8
#endif
#define L ORC_LANES

/* ---- nn helpers ---------------------------------------------------------------------------- */

/* nn.siluInPlace (src/core/nn.zig:399-407): x / (1 + expVec(-x)) over whole vectors, the scalar
 * silu (x / (1 + exp(-x))) over the tail. */
void orc_silu_in_place(float *x, size_t n) {
    size_t i = 0;
    for (; i + L <= n; i += L)
        for (int e = 0; e < L; e++) x[i + e] = x[i + e] / (1.0f + orc_exp_vec(-x[i + e]));
    for (; i < n; i++) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* nn.mulSilu (src/core/nn.zig:410-420): dst = gate * (up / (1 + expVec(-up))). */
void orc_mul_silu(float *dst, const float *gate, const float *up, size_t n) {
    size_t i = 0;
    for (; i + L <= n; i += L)
        for (int e = 0; e < L; e++) {
            const float u = up[i + e];
            dst[i + e] = gate[i + e] * (u / (1.0f + orc_exp_vec(-u)));
        }
    for (; i < n; i++) dst[i] = gate[i] * (up[i] / (1.0f + expf(-up[i])));
}

/* nn.softplus (src/core/nn.zig:516-518). */
float orc_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* nn.clampNonfinite (src/core/nn.zig:522-563): +inf -> the largest finite value, -inf -> the
 * smallest, any remaining infinity (no finite value at all) -> 0; NaN untouched. The lane split
 * of the reference only changes the order of max/min, not the result. */
void orc_clamp_nonfinite(float *v, size_t n) {
    float hi = -INFINITY, lo = INFINITY;
    int any_inf = 0;
    for (size_t i = 0; i < n; i++) {
        const float x = v[i];
        if (isfinite(x)) {
            hi = x > hi ? x : hi;
            lo = x < lo ? x : lo;
        } else if (isinf(x)) {
            any_inf = 1;
        }
    }
    if (!any_inf) return;
    for (size_t i = 0; i < n; i++) {
        float d = v[i];
        if (d == INFINITY) d = hi;
        if (d == -INFINITY) d = lo;
        if (isinf(d)) d = 0;
        v[i] = d;
    }
}

/* ResBlock(.silu).forward (src/core/resblock.zig:63-79); biases may be NULL (bias = false). */
void orc_resblock_silu(size_t threads, float *y, const float *x, size_t rows, const orc_resblock *rb) {
    const size_t in = rb->in, hid = rb->hid, out = rb->out;
    float *h = (float *)malloc(rows * hid * sizeof(float) + 1);
    float *r = (float *)malloc(rows * out * sizeof(float) + 1);
    orc_linear(threads, h, x, rows, rb->hidden_w, hid, in, rb->hidden_b);
    orc_silu_in_place(h, rows * hid);
    orc_linear(threads, y, h, rows, rb->output_w, out, hid, rb->output_b);
    orc_linear(threads, r, x, rows, rb->residual_w, out, in, rb->residual_b);
    orc_add_in_place(y, r, rows * out);
    free(h);
    free(r);
}

/* ---- StatsJob: causal per-patch float64 Welford (src/timestral/model.zig:712-750) ---------- */

typedef struct {
    float *loc, *scale;
    const float *data;
    const uint8_t *obs;
    size_t t, ps;
    double min_scale;
} stats_job;

static void stats_rows(const void *p, size_t r0, size_t r1) {
    const stats_job *j = (const stats_job *)p;
    const size_t t = j->t, ps = j->ps, n = t / ps;
    for (size_t r = r0; r < r1; r++) {
        double cum_w = 0, cum_x = 0, m2 = 0, prev_mean = 0;
        for (size_t pt = 0; pt < n; pt++) {
            for (size_t k = 0; k < ps; k++) {
                const size_t i = pt * ps + k;
                const double w = j->obs[r * t + i] ? 1.0 : 0.0;
                const double x = (double)j->data[r * t + i];
                cum_w += w;
                cum_x += w * x;
                const double den = fmax(cum_w, 1.0);
                const double mean = cum_x / den;
                m2 += (x - prev_mean) * (x - mean) * w;
                prev_mean = mean;
            }
            const double den = fmax(cum_w, 1.0);
            const double variance = m2 / fmax(den - 1.0, 1.0);
            j->loc[r * n + pt] = (float)prev_mean;
            j->scale[r * n + pt] = (float)fmax(sqrt(variance), j->min_scale);
        }
    }
}

void orc_timestral_patch_stats(size_t threads, float *loc, float *scale, const float *data, const uint8_t *obs,
                               size_t rows, size_t t, size_t ps, double min_scale) {
    const stats_job job = {loc, scale, data, obs, t, ps, min_scale};
    orc_for_range_min(threads, rows, 4, &job, stats_rows);
}

/* ---- predictBlock (targets only) -------------------------------------------------------------- */

/* inv_freq of Model.load (src/timestral/model.zig:180-188), applied in runTransformer's tables
 * (:447-463) through orc_timestral_rope_tables. */

/* runTransformer (src/timestral/model.zig:434-482): x (rows, sl, d) in place; roles (vall) in model.Role
 * order (0 target, 1 past, 2 known), cov = any row not a target (Geo.cov). */
static void run_transformer(size_t threads, float *x, const orc_timestral_model *m, size_t rows, size_t vall,
                            size_t ne, size_t l, size_t h, const uint8_t *key_valid, int keys_all_valid,
                            const size_t *first_obs, const uint8_t *roles, int cov) {
    const size_t d = m->d, hid = m->hid, hd = m->hd, nh = m->nh, sl = ne + h, groups = rows / vall;
    const float eps = m->norm_eps;
    float *xn = (float *)malloc(rows * sl * d * sizeof(float));
    float *delta = (float *)malloc(rows * sl * d * sizeof(float));
    float *mlp_h = (float *)malloc(rows * sl * 2 * hid * sizeof(float));
    float *mlp_a = (float *)malloc(rows * sl * hid * sizeof(float));
    float *qkv = (float *)malloc(rows * sl * 3 * d * sizeof(float));
    float *oa = (float *)malloc(rows * sl * d * sizeof(float));
    float *gate = (float *)malloc(rows * sl * d * sizeof(float));
    float *cos_t = (float *)malloc(groups * sl * (hd / 2) * sizeof(float));
    float *sin_t = (float *)malloc(groups * sl * (hd / 2) * sizeof(float));
    orc_timestral_rope_tables(cos_t, sin_t, groups, ne, l, h, hd, m->rope_dim, m->rope_theta, first_obs);
    uint8_t *bidir = (uint8_t *)calloc(rows + 1, 1); /* TimeJob.attend :600: known rows read every valid key */
    for (size_t r = 0; r < rows; r++) bidir[r] = cov && roles[r % vall] == 2;
    for (size_t li = 0; li < m->n_layers; li++) {
        const orc_timestral_layer *ly = &m->layers[li];
        for (int ai = 0; ai < ly->n_attn; ai++) {
            const orc_timestral_attn *a = &ly->attn[ai];
            orc_rms_norm(threads, xn, x, rows * sl, d, a->norm, eps);
            orc_linear(threads, qkv, xn, rows * sl, a->qkv, 3 * d, d, NULL);
            if (a->gate) orc_linear(threads, gate, xn, rows * sl, a->gate, d, d, NULL);
            if (a->is_time) {
                /* timeAttention (:487-519): rope, attend per (row, head), gate, out */
                orc_timestral_rope(threads, qkv, cos_t, sin_t, rows, sl, vall, d, nh, hd);
                orc_timestral_time_attention(threads, qkv, oa, key_valid, keys_all_valid, bidir, rows, ne, l, h, d,
                                             nh, hd);
            } else {
                /* variateAttention (:525-544), with the covariate firewalls when cov */
                orc_timestral_variate_attention(threads, qkv, oa, key_valid, roles, cov, groups, vall, ne, h, d,
                                                nh, hd);
            }
            if (a->gate) orc_mul_sigmoid(oa, oa, gate, rows * sl * d);
            orc_linear(threads, delta, oa, rows * sl, a->out, d, d, NULL);
            orc_add_in_place(x, delta, rows * sl * d);
        }
        orc_rms_norm(threads, xn, x, rows * sl, d, ly->mlp_norm, eps);
        orc_linear(threads, mlp_h, xn, rows * sl, ly->w12, 2 * hid, d, NULL);
        for (size_t i = 0; i < rows * sl; i++)  /* MlpAct.run (:41-46) */
            orc_mul_silu(mlp_a + i * hid, mlp_h + i * 2 * hid, mlp_h + i * 2 * hid + hid, hid);
        orc_linear(threads, delta, mlp_a, rows * sl, ly->w3, d, hid, NULL);
        orc_add_in_place(x, delta, rows * sl * d);
    }
    free(xn); free(delta); free(mlp_h); free(mlp_a); free(qkv); free(oa); free(gate); free(cos_t); free(sin_t);
    free(bidir);
}

/* Model.predictBlock (src/timestral/model.zig:220-432): ctx/obs (rows, t), rows = groups * vall,
 * roles (vall) in model.Role order (0 target, 1 past, 2 known; NULL = every row a target); kf/kfm
 * (rows, h * ps) the known-future values and observations (NULL = blanks). out (groups * n_tgt,
 * h * ps, q): quantiles in data units of the target rows, series by series. */
void orc_timestral_predict_block_cov(size_t threads, float *out, const orc_timestral_model *m, const float *ctx,
                                     const uint8_t *obs, size_t t, size_t groups, size_t vall, size_t h,
                                     const uint8_t *roles_in, const float *kf, const uint8_t *kfm) {
    const size_t ps = m->ps, d = m->d, q = m->q, rows = groups * vall, l = t / ps, hl = h * ps;
    uint8_t *roles = (uint8_t *)calloc(vall + 1, 1);
    int cov = 0;
    size_t n_tgt = 0;
    for (size_t i = 0; i < vall; i++) {
        roles[i] = roles_in ? roles_in[i] : 0;
        cov = cov || roles[i] != 0;
        n_tgt += roles[i] == 0;
    }
    /* The window (:253-273): the context, plus (with covariates) the horizon blanks / known futures. */
    const size_t w = cov ? t + hl : t, n = w / ps;
    float *full = (float *)malloc(rows * w * sizeof(float) + 1);
    uint8_t *full_obs = (uint8_t *)malloc(rows * w + 1);
    for (size_t r = 0; r < rows; r++) {
        memcpy(full + r * w, ctx + r * t, t * sizeof(float));
        memcpy(full_obs + r * w, obs + r * t, t);
        for (size_t j = t; j < w; j++) {
            full[r * w + j] = kf ? kf[r * hl + j - t] : 0.0f;
            full_obs[r * w + j] = kf ? (kfm[r * hl + j - t] != 0) : 0;
        }
    }
    float *loc = (float *)malloc(rows * n * sizeof(float) + 1);
    float *scale = (float *)malloc(rows * n * sizeof(float) + 1);
    orc_timestral_patch_stats(threads, loc, scale, full, full_obs, rows, w, ps, m->minimum_scale);
    const float eps32 = 1.1920929e-07f; /* std.math.floatEps(f32) */
    float *emb_in = (float *)malloc(rows * n * 2 * ps * sizeof(float) + 1);
    for (size_t r = 0; r < rows; r++) {
        const int known = cov && roles[r % vall] == 2;
        /* Known-future rows: whole-window f32 statistics; 0/1 indicator rows skip the asinh (:285-310). */
        float kloc = 0, kscale = 1;
        int binary = 0;
        if (known) {
            float cnt = 0, sum = 0;
            int zero_one = 1, any = 0;
            for (size_t i = 0; i < w; i++)
                if (full_obs[r * w + i]) {
                    const float xv = full[r * w + i];
                    cnt += 1;
                    sum += xv;
                    zero_one = zero_one && (xv == 0 || xv == 1);
                    any = 1;
                }
            kloc = sum / fmaxf(cnt, 1.0f);
            float ss = 0;
            for (size_t i = 0; i < w; i++)
                if (full_obs[r * w + i]) {
                    const float dv = full[r * w + i] - kloc;
                    ss += dv * dv;
                }
            kscale = fmaxf(sqrtf(ss / fmaxf(cnt, 1.0f)), (float)m->minimum_scale);
            binary = zero_one && any;
            if (binary) {
                kloc = 0;
                kscale = 1;
            }
        }
        for (size_t p = 0; p < n; p++) {
            const float lo = known ? kloc : loc[r * n + p];
            const float sc = fmaxf(known ? kscale : scale[r * n + p], eps32);
            float *dst = emb_in + (r * n + p) * 2 * ps;
            for (size_t i = 0; i < ps; i++) {
                const int ob = full_obs[r * w + p * ps + i] != 0;
                float v = 0;
                if (ob) {
                    v = (full[r * w + p * ps + i] - lo) / sc;
                    if (m->use_asinh && !(known && binary)) v = asinhf(v);
                }
                dst[i] = v;
                dst[ps + i] = ob ? 0.0f : 1.0f;
            }
        }
    }
    const size_t ne = n, sl = ne + h;
    float *x = (float *)malloc(rows * sl * d * sizeof(float));
    float *enc = (float *)malloc(rows * ne * d * sizeof(float) + 1);
    orc_resblock_silu(threads, enc, emb_in, rows * ne, &m->patch_proj);
    for (size_t r = 0; r < rows; r++) {
        memcpy(x + r * sl * d, enc + r * ne * d, ne * d * sizeof(float));
        for (size_t j = 0; j < h; j++) memcpy(x + (r * sl + ne + j) * d, m->forecast_query, d * sizeof(float));
    }
    uint8_t *key_valid = (uint8_t *)malloc(rows * ne + 1);
    size_t *first_obs = (size_t *)malloc(groups * sizeof(size_t) + 1);
    const int all_valid =
        orc_timestral_key_valid(key_valid, first_obs, full_obs, rows, vall, ne, ps, m->attend_missing);
    run_transformer(threads, x, m, rows, vall, ne, l, h, key_valid, all_valid, first_obs, roles, cov);

    /* Head on the target rows' decoder tokens (:380-391). */
    const size_t n_out = groups * n_tgt;
    float *dec = (float *)malloc(n_out * h * d * sizeof(float) + 1);
    size_t *out_row = (size_t *)malloc(n_out * sizeof(size_t) + 1);
    for (size_t r = 0, oi = 0; r < rows; r++) {
        if (roles[r % vall] != 0) continue;
        orc_rms_norm(threads, dec + oi * h * d, x + (r * sl + ne) * d, h, d, m->out_norm, m->norm_eps);
        out_row[oi++] = r;
    }
    float *raw = (float *)malloc(n_out * hl * q * sizeof(float) + 1);
    orc_resblock_silu(threads, raw, dec, n_out * h, &m->head);
    const size_t med = m->median;
    float *widths = (float *)calloc(q, sizeof(float));
    for (size_t i = med + 1; i < q; i++) widths[i] = (float)(m->knots[i] - m->knots[i - 1]);
    for (size_t i = 0; i < med; i++) widths[i] = (float)(m->knots[i + 1] - m->knots[i]);
    const float wf = m->quantile_width_factor, big = 3.40282347e38f;
    for (size_t oi = 0; oi < n_out; oi++) {
        const size_t r = out_row[oi];
        /* Anchor frame: the last context patch (patch l - 1 of the window). */
        const float lo = loc[r * n + l - 1], sc = scale[r * n + l - 1];
        for (size_t s = 0; s < hl; s++) {
            const float *rv = raw + (oi * hl + s) * q;
            float *ov = out + (oi * hl + s) * q;
            const float mv = rv[med];
            float acc = 0;
            for (size_t i = med + 1; i < q; i++) {
                const float inc = (wf * widths[i]) * orc_softplus(rv[i]);
                acc += inc;
                ov[i] = fmaxf(-big, fminf(mv + acc, big)); /* std.math.clamp: @max(lo, @min(x, hi)) */
            }
            acc = 0;
            for (size_t i = med; i > 0;) {
                i--;
                const float inc = (wf * widths[i]) * orc_softplus(rv[i]);
                acc += inc;
                ov[i] = fmaxf(-big, fminf(mv - acc, big));
            }
            ov[med] = mv;
            for (size_t i = 0; i < q; i++) {
                const float y = m->use_asinh ? sinhf(ov[i]) : ov[i];
                const float ys = y * sc;
                ov[i] = ys + lo;
            }
            orc_clamp_nonfinite(ov, q);
        }
    }
    free(roles); free(full); free(full_obs); free(loc); free(scale); free(emb_in); free(x); free(enc);
    free(key_valid); free(first_obs); free(dec); free(out_row); free(raw); free(widths);
}

/* Model.predictBlock with every row a target (cov = false): out (rows, h * ps, q). */
void orc_timestral_predict_block(size_t threads, float *out, const orc_timestral_model *m, const float *ctx,
                                 const uint8_t *obs, size_t t, size_t groups, size_t vall, size_t h) {
    orc_timestral_predict_block_cov(threads, out, m, ctx, obs, t, groups, vall, h, NULL, NULL, NULL);
}

/* ---- forecaster ------------------------------------------------------------------------------ */

typedef struct { double w, mean, m2; } welford;

/* welfordCombine (src/timestral/forecaster.zig:567-577). */
static welford welford_combine(welford a, welford b) {
    const double w = a.w + b.w;
    if (w == 0) return (welford){0, 0, 0};
    const double w_safe = w > 2.2250738585072014e-308 ? w : 2.2250738585072014e-308; /* floatMin(f64) */
    const double delta = b.mean - a.mean;
    return (welford){w, a.mean + delta * b.w / w_safe, a.m2 + b.m2 + delta * delta * a.w * b.w / w_safe};
}

/* refineBlock (src/timestral/forecaster.zig:582-662), every row a target: qs (rows, h * ps, q). */
void orc_timestral_refine_block(float *qs, const orc_timestral_model *m, const float *ctx, const uint8_t *obs,
                                size_t rows, size_t t, size_t h) {
    const size_t ps = m->ps, q = m->q, med = m->median, l = t / ps;
    float *loc = (float *)malloc(l * sizeof(float) + 1), *scale = (float *)malloc(l * sizeof(float) + 1);
    const double clip = sqrt((double)3.40282347e38f) / 1e3;
    double *sinh_med = (double *)malloc(h * ps * sizeof(double));
    float *loc_j = (float *)malloc(h * sizeof(float)), *scale_j = (float *)malloc(h * sizeof(float));
    double folded[256];
    for (size_t r = 0; r < rows; r++) {
        const float *row_ctx = ctx + r * t;
        const uint8_t *row_mask = obs + r * t;
        orc_timestral_patch_stats(1, loc, scale, row_ctx, row_mask, 1, t, ps, m->minimum_scale);
        const float loc0 = loc[l - 1], scale0 = scale[l - 1];
        float *block = qs + r * h * ps * q;
        for (size_t s = 0; s < h * ps; s++) sinh_med[s] = ((double)block[s * q + med] - (double)loc0) / (double)scale0;
        welford state = {0, 0, 0};
        for (size_t p = 0; p < l; p++) {
            double cnt = 0, sum = 0;
            for (size_t k = 0; k < ps; k++)
                if (row_mask[p * ps + k]) {
                    cnt += 1;
                    sum += row_ctx[p * ps + k];
                }
            welford pm = {cnt, 0, 0};
            if (cnt > 0) {
                pm.mean = sum / fmax(cnt, 1.0);
                for (size_t k = 0; k < ps; k++)
                    if (row_mask[p * ps + k]) {
                        const double dv = (double)row_ctx[p * ps + k] - pm.mean;
                        pm.m2 += dv * dv;
                    }
            }
            state = welford_combine(state, pm);
        }
        const double offset = state.mean;
        for (size_t j = 0; j < h; j++) {
            const double variance = fmax(state.m2 / fmax(state.w - 1.0, 1.0), 0.0);
            const double sc = fmax(sqrt(variance), m->minimum_scale);
            loc_j[j] = (float)state.mean;
            scale_j[j] = (float)sc;
            double bsum = 0;
            for (size_t k = 0; k < ps; k++) {
                const double v = sinh_med[j * ps + k] * sc + state.mean - offset;
                folded[k] = fmax(-clip, fmin(v, clip)) + offset;
                bsum += folded[k];
            }
            const double bmean = bsum / (double)ps;
            double bm2 = 0;
            for (size_t k = 0; k < ps; k++) bm2 += (folded[k] - bmean) * (folded[k] - bmean);
            state = welford_combine(state, (welford){(double)ps, bmean, bm2});
        }
        loc_j[0] = loc0;
        scale_j[0] = scale0;
        for (size_t s = 0; s < h * ps; s++) {
            float *rowq = block + s * q;
            const float lj = loc_j[s / ps], sj = scale_j[s / ps];
            for (size_t i = 0; i < q; i++) {
                const float a = (rowq[i] - loc0) / scale0;
                const float b = a * sj;
                rowq[i] = b + lj;
            }
            orc_clamp_nonfinite(rowq, q);
        }
    }
    free(loc); free(scale); free(sinh_med); free(loc_j); free(scale_j);
}

/* blockDecode (src/timestral/forecaster.zig:423-563): rows/mask (groups * vall, t_in) padded context,
 * roles (vall) with the v target rows first, kf/kfm (groups * vall, hpad) known futures or NULL; out
 * (groups * v, horizon, q). Re-encodes the whole grown context every block. Feedback: targets carry
 * their median, known covariates their real future, past-only covariates a blank. */
static void block_decode(size_t threads, float *out, const orc_timestral_model *m, const float *rows_in,
                         const uint8_t *mask_in, size_t groups, size_t vall, const uint8_t *roles, size_t v,
                         const float *kf, const uint8_t *kfm, size_t hpad, size_t t_in, size_t horizon,
                         size_t max_context, size_t per_shot, float extreme) {
    const size_t ps = m->ps, q = m->q, med = m->median, nrows = groups * vall, nt = groups * v;
    size_t t = t_in;
    float *ctx = (float *)malloc(nrows * t * sizeof(float) + 1);
    uint8_t *cmask = (uint8_t *)malloc(nrows * t + 1);
    memcpy(ctx, rows_in, nrows * t * sizeof(float));
    memcpy(cmask, mask_in, nrows * t);
    size_t remaining = (horizon + ps - 1) / ps, done = 0;
    while (remaining > 0) {
        const size_t block = per_shot < remaining ? per_shot : remaining, blen = block * ps;
        float *qs = (float *)malloc(nt * blen * q * sizeof(float));
        float *kfb = NULL;
        uint8_t *kfmb = NULL;
        if (kf) {
            kfb = (float *)malloc(nrows * blen * sizeof(float));
            kfmb = (uint8_t *)malloc(nrows * blen);
            for (size_t r = 0; r < nrows; r++) {
                memcpy(kfb + r * blen, kf + r * hpad + done, blen * sizeof(float));
                memcpy(kfmb + r * blen, kfm + r * hpad + done, blen);
            }
        }
        orc_timestral_predict_block_cov(threads, qs, m, ctx, cmask, t, groups, vall, block, roles, kfb, kfmb);
        if (block > 1) /* refineBlock (:582-662) on the target rows g * vall + i, i < v */
            for (size_t g = 0; g < groups; g++)
                for (size_t i = 0; i < v; i++) {
                    const size_t r = g * vall + i;
                    orc_timestral_refine_block(qs + (g * v + i) * blen * q, m, ctx + r * t, cmask + r * t, 1, t, block);
                }
        for (size_t r = 0; r < nt; r++)
            for (size_t s = 0; s < blen; s++) {
                if (done + s >= horizon) break;
                memcpy(out + (r * horizon + done + s) * q, qs + (r * blen + s) * q, q * sizeof(float));
            }
        remaining -= block;
        done += blen;
        if (remaining == 0) {
            free(qs); free(kfb); free(kfmb);
            break;
        }
        const size_t nt_len = t + blen;
        size_t keep_t = nt_len;
        if (nt_len > max_context) keep_t = max_context / ps * ps > ps ? max_context / ps * ps : ps; /* @max(ps, ..) */
        float *nctx = (float *)malloc(nrows * keep_t * sizeof(float));
        uint8_t *nmask = (uint8_t *)malloc(nrows * keep_t);
        const size_t start = nt_len - keep_t, ncopy = start < t ? t - start : 0, s0 = start < t ? 0 : start - t;
        for (size_t g = 0; g < groups; g++) {
            size_t ti = 0;
            for (size_t i = 0; i < vall; i++) {
                const size_t r = g * vall + i, trow = g * v + ti;
                if (ncopy > 0) {
                    memcpy(nctx + r * keep_t, ctx + r * t + start, ncopy * sizeof(float));
                    memcpy(nmask + r * keep_t, cmask + r * t + start, ncopy);
                }
                for (size_t s = s0; s < s0 + (keep_t - ncopy); s++) {
                    const size_t j = s - s0 + ncopy;
                    if (roles[i] == 0) {
                        float mv = qs[(trow * blen + s) * q + med];
                        if (!isfinite(mv) || fabsf(mv) >= extreme) mv = 0;
                        nctx[r * keep_t + j] = mv;
                        nmask[r * keep_t + j] = 1;
                    } else if (roles[i] == 2) {
                        nctx[r * keep_t + j] = kfb[r * blen + s];
                        nmask[r * keep_t + j] = kfmb[r * blen + s];
                    } else {
                        nctx[r * keep_t + j] = 0;
                        nmask[r * keep_t + j] = 0;
                    }
                }
                if (roles[i] == 0) ti++;
            }
        }
        free(ctx); free(cmask); free(qs); free(kfb); free(kfmb);
        ctx = nctx;
        cmask = nmask;
        t = keep_t;
    }
    free(ctx);
    free(cmask);
}

/* forecastRaw (src/timestral/forecaster.zig:303-421): inputs/observed (b, v, t0); past (b, n_past,
 * t0) and known (b, n_known, t0 + horizon) covariates, NaN = missing, either may be NULL with a
 * count of 0; out (b, v, horizon, q). Returns 0, or 1 for a NaN forecast (error.DegenerateInput). */
static int forecast_raw(size_t threads, float *out, const orc_timestral_model *m, const float *inputs,
                        const uint8_t *observed, size_t b, size_t v, size_t t0, size_t horizon, const float *past,
                        size_t n_past, const float *known, size_t n_known, size_t max_context, size_t per_shot,
                        float cap_k, float extreme) {
    const size_t ps = m->ps, q = m->q, vall = v + n_past + n_known, nrows = b * vall;
    uint8_t *roles = (uint8_t *)malloc(vall + 1);
    for (size_t i = 0; i < vall; i++) roles[i] = i < v ? 0 : i < v + n_past ? 1 : 2;
    const size_t keep = t0 < max_context ? t0 : max_context, t = (keep + ps - 1) / ps * ps;
    const size_t hpad = (horizon + ps - 1) / ps * ps;
    float *rows = (float *)calloc(nrows * t + 1, sizeof(float));
    uint8_t *mask = (uint8_t *)calloc(nrows * t + 1, 1);
    float *kf = (float *)calloc(nrows * hpad + 1, sizeof(float));
    uint8_t *kfm = (uint8_t *)calloc(nrows * hpad + 1, 1);
    for (size_t s = 0; s < b; s++)
        for (size_t i = 0; i < vall; i++) {
            const size_t r = s * vall + i;
            float last = 0;
            int seen = 0;
            for (size_t j = 0; j < t0; j++) {
                float val;
                int ob;
                if (roles[i] == 0) { /* forward-fill the target; leading gaps stay 0 */
                    const size_t idx = (s * v + i) * t0 + j;
                    if (observed[idx]) {
                        last = inputs[idx];
                        seen = 1;
                    }
                    val = seen ? last : 0;
                    ob = observed[idx] != 0;
                } else {
                    const float xv = roles[i] == 1 ? past[(s * n_past + (i - v)) * t0 + j]
                                                   : known[(s * n_known + (i - v - n_past)) * (t0 + horizon) + j];
                    ob = !isnan(xv);
                    val = ob ? xv : 0;
                }
                if (j >= t0 - keep) {
                    const size_t dst = r * t + (t - keep) + (j - (t0 - keep));
                    rows[dst] = val;
                    mask[dst] = (uint8_t)ob;
                }
            }
            if (roles[i] == 2)
                for (size_t j = 0; j < horizon; j++) {
                    const float xv = known[(s * n_known + (i - v - n_past)) * (t0 + horizon) + t0 + j];
                    kfm[r * hpad + j] = !isnan(xv);
                    kf[r * hpad + j] = isnan(xv) ? 0 : xv;
                }
        }
    block_decode(threads, out, m, rows, mask, b, vall, roles, v, n_known ? kf : NULL, n_known ? kfm : NULL, hpad, t,
                 horizon, max_context, per_shot, extreme);
    if (cap_k > 0) {
        const size_t n = t / ps;
        float *loc = (float *)malloc(n * sizeof(float) + 1), *scale = (float *)malloc(n * sizeof(float) + 1);
        for (size_t s = 0; s < b; s++)
            for (size_t i = 0; i < v; i++) {
                const size_t r = s * vall + i, o = s * v + i;
                orc_timestral_patch_stats(1, loc, scale, rows + r * t, mask + r * t, 1, t, ps, m->minimum_scale);
                float mx = -INFINITY, mn = INFINITY;
                for (size_t j = 0; j < t; j++)
                    if (mask[r * t + j]) {
                        mx = rows[r * t + j] > mx ? rows[r * t + j] : mx;
                        mn = rows[r * t + j] < mn ? rows[r * t + j] : mn;
                    }
                if (isinf(mx)) mx = 0;
                if (isinf(mn)) mn = 0;
                const float a = scale[n - 1] * cap_k, lo = mn - a, hi = mx + a;
                for (size_t k = 0; k < horizon * q; k++)  /* std.math.clamp: @max(lo, @min(x, hi)) */
                    out[o * horizon * q + k] = fmaxf(lo, fminf(out[o * horizon * q + k], hi));
            }
        free(loc);
        free(scale);
    }
    free(rows); free(mask); free(kf); free(kfm); free(roles);
    for (size_t i = 0; i < b * v * horizon * q; i++)
        if (isnan(out[i])) return 1;
    return 0;
}

/* forecaster.forecast + finish (src/timestral/forecaster.zig:57-180) with numeric covariates (past
 * (b, n_past, t), known (b, n_known, t + horizon), NaN = missing). Returns 0, 1 (a NaN forecast) or 2
 * (asymmetric quantile levels with symmetric averaging). The mirrored pass negates the context and
 * every covariate row (:112-121). */
int orc_timestral_forecast_cov(size_t threads, float *out, const orc_timestral_model *m, const float *inputs,
                               const uint8_t *observed, size_t b, size_t v, size_t t, size_t horizon,
                               const float *past, size_t n_past, const float *known, size_t n_known,
                               size_t max_context, size_t per_shot, float cap_k, float extreme, int symmetric,
                               int clip_nonnegative) {
    const size_t q = m->q;
    if (max_context == 0) max_context = m->context_length;
    if (per_shot > m->block_size) per_shot = m->block_size;
    int rc;
    if (symmetric) {
        for (size_t i = 0; i < q; i++)
            if (fabs(m->knots[i] + m->knots[q - 1 - i] - 1.0) > 1e-9) return 2;
        float *neg = (float *)malloc(b * v * t * sizeof(float) + 1);
        for (size_t i = 0; i < b * v * t; i++) neg[i] = -inputs[i];
        float *negp = (float *)malloc(b * n_past * t * sizeof(float) + 1);
        float *negk = (float *)malloc(b * n_known * (t + horizon) * sizeof(float) + 1);
        for (size_t i = 0; i < b * n_past * t; i++) negp[i] = -past[i];
        for (size_t i = 0; i < b * n_known * (t + horizon); i++) negk[i] = -known[i];
        float *mir = (float *)malloc(b * v * horizon * q * sizeof(float));
        rc = forecast_raw(threads, out, m, inputs, observed, b, v, t, horizon, past, n_past, known, n_known,
                          max_context, per_shot, cap_k, extreme);
        const int rc2 = forecast_raw(threads, mir, m, neg, observed, b, v, t, horizon, negp, n_past, negk, n_known,
                                     max_context, per_shot, cap_k, extreme);
        free(negp);
        free(negk);
        if (rc == 0) rc = rc2;
        for (size_t i = 0; i < b * v * horizon; i++)
            for (size_t j = 0; j < q; j++) {
                const float s = out[i * q + j] + -mir[i * q + q - 1 - j];
                out[i * q + j] = 0.5f * s;
            }
        free(neg);
        free(mir);
    } else {
        rc = forecast_raw(threads, out, m, inputs, observed, b, v, t, horizon, past, n_past, known, n_known,
                          max_context, per_shot, cap_k, extreme);
    }
    if (rc != 0) return rc;
    if (clip_nonnegative)
        for (size_t r = 0; r < b * v; r++) {
            int any = 0, all_nonneg = 1;
            for (size_t i = 0; i < t; i++)
                if (observed[r * t + i] && isfinite(inputs[r * t + i])) {
                    any = 1;
                    all_nonneg = all_nonneg && inputs[r * t + i] >= 0;
                }
            if (any && all_nonneg)
                for (size_t i = 0; i < horizon * q; i++) {
                    float *x = out + r * horizon * q + i;
                    *x = fmaxf(*x, 0); /* @max(x, 0) */
                }
        }
    return 0;
}

/* forecaster.forecast without covariates. */
int orc_timestral_forecast(size_t threads, float *out, const orc_timestral_model *m, const float *inputs,
                           const uint8_t *observed, size_t b, size_t v, size_t t, size_t horizon, size_t max_context,
                           size_t per_shot, float cap_k, float extreme, int symmetric, int clip_nonnegative) {
    return orc_timestral_forecast_cov(threads, out, m, inputs, observed, b, v, t, horizon, NULL, 0, NULL, 0,
                                      max_context, per_shot, cap_k, extreme, symmetric, clip_nonnegative);
}

/* ---- categorical covariates (src/timestral/forecaster.zig:201-301) --------------------------- */

static int orc_cmp_f64(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return x < y ? -1 : x > y ? 1 : 0;
}

/* slotOf (:292-301): index of code in the sorted categories, or -1 for NaN and unknown codes. */
static long orc_slot_of(const double *cats, size_t nc, double code) {
    if (isnan(code)) return -1;
    size_t lo = 0, hi = nc;
    while (lo < hi) {
        const size_t mid = lo + (hi - lo) / 2;
        if (cats[mid] < code) lo = mid + 1;
        else hi = mid;
    }
    return lo < nc && cats[lo] == code ? (long)lo : -1;
}

/* targetEncode (:243-289), smooth = 1: past codes (t of them) and optional future codes. */
static void orc_target_encode(const double *target, const double *past, size_t t, const double *future,
                              size_t nf, float *out_past, float *out_future) {
    const double smooth = 1.0;
    double item_count = 0, item_sum = 0;
    for (size_t i = 0; i < t; i++)
        if (isfinite(target[i])) {
            item_count += 1;
            item_sum += target[i];
        }
    const double item_mean = item_count > 0 ? item_sum / item_count : 0.0;
    double *cats = (double *)malloc((t + 1) * sizeof(double));
    size_t n = 0;
    for (size_t i = 0; i < t; i++)
        if (isfinite(past[i])) cats[n++] = past[i];
    qsort(cats, n, sizeof(double), orc_cmp_f64);
    size_t nc = 0;
    for (size_t i = 0; i < n; i++)
        if (i == 0 || cats[i] != cats[nc - 1]) cats[nc++] = cats[i];
    double *sums = (double *)calloc(nc + 1, sizeof(double));
    double *counts = (double *)calloc(nc + 1, sizeof(double));
    for (size_t i = 0; i < t; i++) {
        if (!isfinite(target[i])) continue;
        const long sl = orc_slot_of(cats, nc, past[i]);
        const size_t slot = sl < 0 ? nc : (size_t)sl;
        sums[slot] += target[i];
        counts[slot] += 1;
    }
    for (size_t i = 0; i < t; i++) {
        const long sl = orc_slot_of(cats, nc, past[i]);
        const size_t slot = sl < 0 ? nc : (size_t)sl;
        out_past[i] = (float)((smooth * item_mean + sums[slot]) / (smooth + counts[slot]));
    }
    for (size_t i = 0; i < nf; i++) {
        const double cv = future[i];
        double v;
        if (isnan(cv)) {
            v = (smooth * item_mean + sums[nc]) / (smooth + counts[nc]);
        } else {
            const long sl = orc_slot_of(cats, nc, cv);
            v = sl >= 0 ? (smooth * item_mean + sums[sl]) / (smooth + counts[sl]) : item_mean;
        }
        out_future[i] = (float)v;
    }
    free(cats);
    free(sums);
    free(counts);
}

/* encodingTarget + encodeCategorical (:201-238): codes (b, c, len) -> out (b, c, len). With v == 1
 * every code row is target-encoded against the forward-filled target over the last max_context
 * steps (NaN before the first observation and outside the window), and a missing code where the
 * target is NaN stays NaN; otherwise the codes pass through as f32. */
void orc_timestral_encode_categorical(float *out, const double *codes, size_t b, size_t c, size_t len,
                                      const float *inputs, const uint8_t *observed, size_t v, size_t t,
                                      size_t max_context) {
    double *target = (double *)malloc(t * sizeof(double));
    for (size_t s = 0; s < b; s++) {
        if (v == 1) {
            int started = 0;
            float last = 0;
            for (size_t i = 0; i < t; i++) {
                if (observed[s * t + i]) {
                    started = 1;
                    last = inputs[s * t + i];
                }
                const int in_window = t <= max_context || i >= t - max_context;
                target[i] = started && in_window ? (double)last : NAN;
            }
        }
        for (size_t j = 0; j < c; j++) {
            const double *row = codes + (s * c + j) * len;
            float *dst = out + (s * c + j) * len;
            if (v != 1) {
                for (size_t i = 0; i < len; i++) dst[i] = (float)row[i];
                continue;
            }
            orc_target_encode(target, row, t, len > t ? row + t : NULL, len > t ? len - t : 0, dst,
                              len > t ? dst + t : NULL);
            for (size_t i = 0; i < t; i++)
                if (isnan(target[i]) && isnan(row[i])) dst[i] = NAN;
        }
    }
    free(target);
}
