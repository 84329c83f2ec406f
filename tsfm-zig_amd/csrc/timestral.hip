// Timestral forecaster pieces that sit between the matrix-core launches (gfx950): the context
// preparation of forecastRaw, the causal per-patch statistics and patch features of predictBlock,
// the RoPE tables, the gates, the monotone quantile head, refineBlock's frames, the median
// feedback of blockDecode, and the final cap / symmetric average / clip.
//
// Reference: src/timestral/model.zig (predictBlock :220-432, runTransformer :434-482, StatsJob
// :712-750) and src/timestral/forecaster.zig (forecast :57-180, forecastRaw :303-421, blockDecode
// :423-563, refineBlock :582-662), for series of target variates with optional numeric past-only
// and known-future covariate rows (the window, the known rows' statistics and the role feedback).
//
// The sequential recurrences of the reference (the float64 Welford of every row, the fold of
// refineBlock) run one thread per row in the reference's order, so they give the reference's
// values; a row's state is kept between decode blocks and continued over the appended steps,
// which is the same sequence of operations as recomputing the grown row from its start.
#include "common.hpp"
#include "launch.hpp"

// Products and sums are rounded one at a time, as in the reference's scalar and vector code.
#pragma clang fp contract(off)

namespace tsfm {
namespace {

__device__ __forceinline__ double fmax_d(double a, double b) { return fmax(a, b); }

// forecastRaw's rows (src/timestral/forecaster.zig:321-379). Row r = g * vall + i of group g (g <
// batch: forward pass, else the mirrored pass of series g - batch, every value negated,
// forecast.zig:112-121); i < V targets (forward-filled, leading gaps 0), then n_past past-only
// and n_known known-future covariates (NaN = missing). Keep the last `keep` steps, left-pad to t;
// known rows also write their horizon values to kf/kfm (rows, hpad). Also the clip flag of each
// target input row (finish, :163-178).
__global__ void ts_context(const TsContextParams p) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= p.rows) return;
    const int g = r / p.vall, i = r % p.vall;
    const bool mirror = g >= p.batch;
    const int sidx = mirror ? g - p.batch : g;
    const float sign = mirror ? -1.f : 1.f;
    const int t0 = p.t0, keep = p.keep, t = p.t;
    float* c = p.ctx + (int64_t)r * p.cap_t;
    uint8_t* mk = p.mask + (int64_t)r * p.cap_t;
    for (int j = 0; j < t - keep; j++) {
        c[j] = 0.f;
        mk[j] = 0;
    }
    if (i >= p.V) {
        const bool known = i >= p.V + p.n_past;
        const float* x = known ? p.known + ((int64_t)sidx * p.n_known + (i - p.V - p.n_past)) * (t0 + p.horizon)
                               : p.past + ((int64_t)sidx * p.n_past + (i - p.V)) * t0;
        for (int j = t0 - keep; j < t0; j++) {
            const float v = sign * x[j];
            const bool ob = !isnan(v);
            const int dst = (t - keep) + (j - (t0 - keep));
            c[dst] = ob ? v : 0.f;
            mk[dst] = ob ? 1 : 0;
        }
        if (known)
            for (int j = 0; j < p.hpad; j++) {
                const float v = j < p.horizon ? sign * x[t0 + j] : 0.f;
                const bool ob = j < p.horizon && !isnan(v);
                p.kf[(int64_t)r * p.hpad + j] = ob ? v : 0.f;
                p.kfm[(int64_t)r * p.hpad + j] = ob ? 1 : 0;
            }
        return;
    }
    const int src = sidx * p.V + i;
    const float* x = p.inputs + (int64_t)src * t0;
    const uint8_t* o = p.observed + (int64_t)src * t0;
    float last = 0.f;
    bool seen = false, any = false, all_nonneg = true;
    for (int j = 0; j < t0; j++) {
        const float v = sign * x[j];
        const bool ob = o[j] != 0;
        if (ob) {
            last = v;
            seen = true;
            if (isfinite(x[j])) {
                any = true;
                all_nonneg = all_nonneg && x[j] >= 0.f;
            }
        }
        if (j >= t0 - keep) {
            const int dst = (t - keep) + (j - (t0 - keep));
            c[dst] = seen ? last : 0.f;
            mk[dst] = ob ? 1 : 0;
        }
    }
    if (!mirror) p.nonneg[src] = any && all_nonneg;
}

// predictBlock's window with covariates (model.zig:253-273): steps [t, t + blen) of every row are
// the block's known futures (known rows, from step `done` of kf) or blanks (targets and past-only
// rows; the targets' blanks become medians after the block).
__global__ void ts_window(float* ctx, uint8_t* mask, int cap_t, int t, int blen, const float* kf,
                          const uint8_t* kfm, int hpad, int done, int vall, int known_from, int rows) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * blen) return;
    const int r = (int)(idx / blen), j = (int)(idx % blen);
    const bool known = r % vall >= known_from;
    ctx[(int64_t)r * cap_t + t + j] = known ? kf[(int64_t)r * hpad + done + j] : 0.f;
    mask[(int64_t)r * cap_t + t + j] = known ? kfm[(int64_t)r * hpad + done + j] : 0;
}

// Known-future rows' statistics (model.zig:283-310): float32 mean and population std of the
// observed steps of the whole window [0, w), at least min_scale; a row of only 0/1 values is
// neither shifted nor scaled and skips the asinh. Written over every patch of the row's loc and
// scale; other rows keep their causal statistics. One thread per row, the reference's order.
__global__ void ts_known_stats(const float* ctx, const uint8_t* mask, int cap_t, int w, int ps, int rows, int vall,
                               int known_from, float min_scale, float* loc, float* scale, int cap_p,
                               uint8_t* no_asinh) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    if (r % vall < known_from) {
        no_asinh[r] = 0;
        return;
    }
    const float* x = ctx + (int64_t)r * cap_t;
    const uint8_t* o = mask + (int64_t)r * cap_t;
    float cnt = 0.f, sum = 0.f;
    bool zero_one = true, any = false;
    for (int i = 0; i < w; i++)
        if (o[i]) {
            cnt += 1.f;
            sum += x[i];
            zero_one = zero_one && (x[i] == 0.f || x[i] == 1.f);
            any = true;
        }
    float kloc = sum / fmaxf(cnt, 1.f);
    float ss = 0.f;
    for (int i = 0; i < w; i++)
        if (o[i]) {
            const float dv = x[i] - kloc;
            ss += dv * dv;
        }
    float kscale = fmaxf(sqrtf(ss / fmaxf(cnt, 1.f)), min_scale);
    const bool binary = zero_one && any;
    if (binary) {
        kloc = 0.f;
        kscale = 1.f;
    }
    for (int pt = 0; pt < w / ps; pt++) {
        loc[(int64_t)r * cap_p + pt] = kloc;
        scale[(int64_t)r * cap_p + pt] = kscale;
    }
    no_asinh[r] = binary ? 1 : 0;
}

}  // namespace

hipError_t launch_ts_context(const TsContextParams& p, hipStream_t s) {
    hipLaunchKernelGGL(ts_context, dim3((unsigned)((p.rows + 63) / 64)), dim3(64), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_ts_window(float* ctx, uint8_t* mask, int cap_t, int t, int blen, const float* kf, const uint8_t* kfm,
                            int hpad, int done, int vall, int known_from, int rows, hipStream_t s) {
    const int64_t n = (int64_t)rows * blen;
    hipLaunchKernelGGL(ts_window, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ctx, mask, cap_t, t, blen, kf,
                       kfm, hpad, done, vall, known_from, rows);
    return hipGetLastError();
}

hipError_t launch_ts_known_stats(const float* ctx, const uint8_t* mask, int cap_t, int w, int ps, int rows, int vall,
                                 int known_from, float min_scale, float* loc, float* scale, int cap_p,
                                 uint8_t* no_asinh, hipStream_t s) {
    hipLaunchKernelGGL(ts_known_stats, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, s, ctx, mask, cap_t, w, ps,
                       rows, vall, known_from, min_scale, loc, scale, cap_p, no_asinh);
    return hipGetLastError();
}

namespace {

// StatsJob (src/timestral/model.zig:712-750) continued from step `from` (a patch boundary) to t,
// from the row's saved state (st: cum_w, cum_x, m2, prev_mean; zero when from == 0): loc and
// scale of patches [from / ps, t / ps). In the same pass: key validity of those patches
// (model.zig:343-357: observed, or with attend_missing any patch after the row's first observed
// one), the row's first observed patch (-1 if none yet), and refineBlock's fold of the context's
// per-patch moments (forecaster.zig:613-631) into fold (w, mean, m2).
__global__ void ts_stats(const TsStatsParams p) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= p.rows) return;
    const float* x = p.ctx + (int64_t)r * p.cap_t;
    const uint8_t* o = p.mask + (int64_t)r * p.cap_t;
    double* st = p.state + (int64_t)r * 4;
    double* fo = p.fold + (int64_t)r * 3;
    double cum_w = 0, cum_x = 0, m2 = 0, prev_mean = 0;
    double fw = 0, fmean = 0, fm2 = 0;
    int first = -1;
    if (p.from > 0) {
        cum_w = st[0]; cum_x = st[1]; m2 = st[2]; prev_mean = st[3];
        fw = fo[0]; fmean = fo[1]; fm2 = fo[2];
        first = p.row_first[r];
    }
    const int ps = p.ps;
    for (int pt = p.from / ps; pt < p.t / ps; pt++) {
        bool ob_any = false;
        double cnt = 0, sum = 0;
        for (int k = 0; k < ps; k++) {
            const int i = pt * ps + k;
            const bool ob = o[i] != 0;
            const double w = ob ? 1.0 : 0.0;
            const double xv = (double)x[i];
            cum_w += w;
            cum_x += w * xv;
            const double den = fmax_d(cum_w, 1.0);
            const double mean = cum_x / den;
            m2 += (xv - prev_mean) * (xv - mean) * w;
            prev_mean = mean;
            if (ob) {
                ob_any = true;
                cnt += 1;
                sum += (double)x[i];
            }
        }
        const double den = fmax_d(cum_w, 1.0);
        const double variance = m2 / fmax_d(den - 1.0, 1.0);
        p.loc[(int64_t)r * p.cap_p + pt] = (float)prev_mean;
        p.scale[(int64_t)r * p.cap_p + pt] = (float)fmax_d(sqrt(variance), p.min_scale);
        if (ob_any && first < 0) first = pt;
        p.key_valid[(int64_t)r * p.cap_p + pt] = (uint8_t)(p.attend_missing ? (ob_any || first >= 0) : ob_any);
        // refineBlock's per-patch moments, combined with welfordCombine (forecaster.zig:567-577)
        double pm_mean = 0, pm_m2 = 0;
        if (cnt > 0) {
            pm_mean = sum / fmax_d(cnt, 1.0);
            for (int k = 0; k < ps; k++)
                if (o[pt * ps + k]) {
                    const double dv = (double)x[pt * ps + k] - pm_mean;
                    pm_m2 += dv * dv;
                }
        }
        const double w = fw + cnt;
        if (w == 0) {
            fw = 0; fmean = 0; fm2 = 0;
        } else {
            const double w_safe = fmax_d(w, 2.2250738585072014e-308);
            const double delta = pm_mean - fmean;
            const double nm = fmean + delta * cnt / w_safe;
            const double n2 = fm2 + pm_m2 + delta * delta * fw * cnt / w_safe;
            fw = w; fmean = nm; fm2 = n2;
        }
    }
    st[0] = cum_w; st[1] = cum_x; st[2] = m2; st[3] = prev_mean;
    fo[0] = fw; fo[1] = fmean; fo[2] = fm2;
    p.row_first[r] = first;
}

// predictBlock's patch features (model.zig:281-328) of patches [p0, l): values normalised by their
// patch's statistics (asinh'd unless the row's no_asinh flag is set), then the missing-step mask.
__global__ void ts_features(const float* ctx, const uint8_t* mask, int cap_t, const float* loc, const float* scale,
                            int cap_p, int rows, int p0, int l, int ps, int use_asinh, const uint8_t* no_asinh,
                            float* feats) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int np = l - p0;
    if (idx >= (int64_t)rows * np * ps) return;
    const int i = (int)(idx % ps);
    const int64_t rp = idx / ps;
    const int r = (int)(rp / np), pt = p0 + (int)(rp % np);
    const float lo = loc[(int64_t)r * cap_p + pt];
    const float sc = fmaxf(scale[(int64_t)r * cap_p + pt], 1.1920929e-07f);  // @max(scale, floatEps(f32))
    const int64_t at = (int64_t)r * cap_t + pt * ps + i;
    const bool ob = mask[at] != 0;
    float v = 0.f;
    if (ob) {
        v = (ctx[at] - lo) / sc;
        if (use_asinh && !(no_asinh != nullptr && no_asinh[r])) v = asinhf(v);
    }
    float* f = feats + rp * 2 * ps;
    f[i] = v;
    f[ps + i] = ob ? 0.f : 1.f;
}

// First observed patch of each group (model.zig:343-360: over the group's rows, 0 when none) and
// the RoPE tables of runTransformer (:447-463) for token indices [0, n_tok): encoder token p at time
// p, decoder token ne + j at time l + j = its index minus shift (ne - l: 0 without covariates, so
// one table serves every block; the horizon's patches with covariates).
__global__ void ts_rope_tables(const int* row_first, int vall, int n_tok, int ne, int shift, TsRope rp, float* cos_t,
                               float* sin_t, int* first_obs) {
    const int g = blockIdx.y;
    int first = 0x7fffffff;
    for (int i = 0; i < vall; i++) {
        const int f = row_first[g * vall + i];
        if (f >= 0 && f < first) first = f;
    }
    if (first == 0x7fffffff) first = 0;
    if (blockIdx.x == 0 && threadIdx.x == 0) first_obs[g] = first;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)n_tok * 32) return;
    const int tok = (int)(idx / 32), i = (int)(idx % 32);
    const float pos = (float)((tok < ne ? tok : tok - shift) - first);
    const float ang = rp.inv_freq[i] * pos;
    const int64_t at = ((int64_t)g * n_tok + tok) * 32 + i;
    cos_t[at] = cosf(ang);
    sin_t[at] = sinf(ang);
}

// [encoder tokens; decoder tokens] of each row: x[r, i] = emb[r, i] for i < m, the forecast query
// for the h decoder tokens (model.zig:333-341).
__global__ void ts_assemble(const float* emb, const float* query, float* x, int rows, int m, int h, int d) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int sl = m + h, d4 = d / 4;
    if (idx >= (int64_t)rows * sl * d4) return;
    const int c = (int)(idx % d4) * 4;
    const int64_t rt = idx / d4;
    const int r = (int)(rt / sl), tok = (int)(rt % sl);
    const f32x4 v = tok < m ? ld4(emb + ((int64_t)r * m + tok) * d + c) : ld4(query + c);
    st4(x + rt * d + c, v);
}

// nn.mulSigmoid over whole vectors (src/core/nn.zig:423-433): o = o / (1 + exp(-g)).
__global__ void ts_mul_sigmoid(float* o, const float* g, int64_t n4) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n4) return;
    const f32x4 x = ld4(o + 4 * idx), gv = ld4(g + 4 * idx);
    st4(o + 4 * idx, f32x4{x[0] / (1.f + expf(-gv[0])), x[1] / (1.f + expf(-gv[1])), x[2] / (1.f + expf(-gv[2])),
                           x[3] / (1.f + expf(-gv[3]))});
}

// The bf16 time-attention output widened to the f32 buffer the out projection reads, with the
// sigmoid gate of timeAttention (model.zig:517, nn.mulSigmoid) applied as in ts_mul_sigmoid when g is
// given.
__global__ void ts_from_bf16(const uint16_t* oh, const float* g, float* o, int64_t n4) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n4) return;
    const u32x2 w = *reinterpret_cast<const u32x2*>(oh + 4 * idx);
    f32x4 x = {__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u), __uint_as_float(w[1] << 16),
               __uint_as_float(w[1] & 0xffff0000u)};
    if (g != nullptr) {
        const f32x4 gv = ld4(g + 4 * idx);
        x = f32x4{x[0] / (1.f + expf(-gv[0])), x[1] / (1.f + expf(-gv[1])), x[2] / (1.f + expf(-gv[2])),
                  x[3] / (1.f + expf(-gv[3]))};
    }
    st4(o + 4 * idx, x);
}

// MlpAct.run (model.zig:40-46) with nn.mulSilu (src/core/nn.zig:410-420): a[t, i] = gate * silu(up)
// with gate = h[t, i], up = h[t, hid + i].
__global__ void ts_mul_silu(const float* hbuf, float* a, int64_t tokens, int hid) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int h4 = hid / 4;
    if (idx >= tokens * h4) return;
    const int64_t t = idx / h4;
    const int c = (int)(idx % h4) * 4;
    const f32x4 g = ld4(hbuf + t * 2 * hid + c), u = ld4(hbuf + t * 2 * hid + hid + c);
    st4(a + t * hid + c, f32x4{g[0] * (u[0] / (1.f + expf(-u[0]))), g[1] * (u[1] / (1.f + expf(-u[1]))),
                               g[2] * (u[2] / (1.f + expf(-u[2]))), g[3] * (u[3] / (1.f + expf(-u[3])))});
}

// nn.clampNonfinite (src/core/nn.zig:522-563) of one quantile vector.
__device__ void clamp_nonfinite(float* v, int q) {
    float hi = -INFINITY, lo = INFINITY;
    bool any_inf = false;
    for (int i = 0; i < q; i++) {
        if (isfinite(v[i])) {
            hi = fmaxf(hi, v[i]);
            lo = fminf(lo, v[i]);
        } else if (isinf(v[i])) {
            any_inf = true;
        }
    }
    if (!any_inf) return;
    for (int i = 0; i < q; i++) {
        float d = v[i];
        if (d == INFINITY) d = hi;
        if (d == -INFINITY) d = lo;
        if (isinf(d)) d = 0.f;
        v[i] = d;
    }
}

// The monotone quantile head of predictBlock (model.zig:391-431): per (row, step) the median is
// free and the other levels fan out by cumulative softplus increments scaled by the knot widths,
// then back to data units with the last context patch's (loc, scale). raw: per decoder token
// ps * q outputs ordered (step, level); qs (rows, h * ps, q).
__global__ void ts_head_finish(const float* raw, const float* loc, const float* scale, int cap_p, int l, int rows,
                               int h, TsHead hp, float* qs) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int hl = h * hp.ps, q = hp.q, m = hp.median;
    if (idx >= (int64_t)rows * hl) return;
    const int r = (int)(idx / hl);
    const float* rv = raw + idx * q;  // token j = s / ps, step i = s % ps: (r * h + j) * ps * q + i * q
    float ov[32];
    const float med = rv[m], big = 3.40282347e38f;
    float acc = 0.f;
    for (int i = m + 1; i < q; i++) {
        const float x = rv[i];
        const float sp = x > 20.f ? x : log1pf(expf(x));
        acc += (hp.wf * hp.widths[i]) * sp;
        ov[i] = fmaxf(-big, fminf(med + acc, big));
    }
    acc = 0.f;
    for (int i = m - 1; i >= 0; i--) {
        const float x = rv[i];
        const float sp = x > 20.f ? x : log1pf(expf(x));
        acc += (hp.wf * hp.widths[i]) * sp;
        ov[i] = fmaxf(-big, fminf(med - acc, big));
    }
    ov[m] = med;
    const float lo = loc[(int64_t)r * cap_p + l - 1], sc = scale[(int64_t)r * cap_p + l - 1];
    for (int i = 0; i < q; i++) {
        const float y = hp.use_asinh ? sinhf(ov[i]) : ov[i];
        const float ys = y * sc;
        ov[i] = ys + lo;
    }
    clamp_nonfinite(ov, q);
    float* o = qs + idx * q;
    for (int i = 0; i < q; i++) o[i] = ov[i];
}

// refineBlock's frames (src/timestral/forecaster.zig:602-652), one thread per row: fold the block's
// medians (in the context's last-patch frame) patch by patch into the context's Welford state;
// frames[r, j] = (loc_j, scale_j), patch 0 keeping (loc0, scale0).
__global__ void ts_refine_frames(const float* qs, const float* loc, const float* scale, int cap_p, int l,
                                 const double* fold, int rows, int h, int ps, int q, int median, double min_scale,
                                 float* frames) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float loc0 = loc[(int64_t)r * cap_p + l - 1], scale0 = scale[(int64_t)r * cap_p + l - 1];
    double w = fold[r * 3 + 0], mean = fold[r * 3 + 1], m2 = fold[r * 3 + 2];
    const double clip = sqrt((double)3.40282347e38f) / 1e3, offset = mean;
    const float* block = qs + (int64_t)r * h * ps * q;
    float* fr = frames + (int64_t)r * h * 2;
    for (int j = 0; j < h; j++) {
        const double variance = fmax_d(m2 / fmax_d(w - 1.0, 1.0), 0.0);
        const double sc = fmax_d(sqrt(variance), min_scale);
        fr[2 * j] = (float)mean;
        fr[2 * j + 1] = (float)sc;
        // The block's medians of patch j mapped into this frame (computed twice: once for their
        // mean, once for the squared deviations).
        auto folded = [&](int k) {
            const double sm = ((double)block[(j * ps + k) * q + median] - (double)loc0) / (double)scale0;
            const double v = sm * sc + mean - offset;
            return fmax_d(-clip, fmin(v, clip)) + offset;
        };
        double bsum = 0;
        for (int k = 0; k < ps; k++) bsum += folded(k);
        const double bmean = bsum / (double)ps;
        double bm2 = 0;
        for (int k = 0; k < ps; k++) {
            const double f = folded(k);
            bm2 += (f - bmean) * (f - bmean);
        }
        // welfordCombine(state, (ps, bmean, bm2))
        const double bw = (double)ps, nw = w + bw;
        if (nw == 0) {
            w = 0; mean = 0; m2 = 0;
        } else {
            const double w_safe = fmax_d(nw, 2.2250738585072014e-308);
            const double delta = bmean - mean;
            const double nm = mean + delta * bw / w_safe;
            const double n2 = m2 + bm2 + delta * delta * w * bw / w_safe;
            w = nw; mean = nm; m2 = n2;
        }
    }
    fr[0] = loc0;
    fr[1] = scale0;
}

// refineBlock's rescale (forecaster.zig:653-659): (x - loc0) / scale0 * scale_j + loc_j, then
// nn.clampNonfinite of each step's levels.
__global__ void ts_refine_apply(float* qs, const float* frames, int rows, int h, int ps, int q) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int hl = h * ps;
    if (idx >= (int64_t)rows * hl) return;
    const int r = (int)(idx / hl), s = (int)(idx % hl);
    const float* fr = frames + (int64_t)r * h * 2;
    const float loc0 = fr[0], scale0 = fr[1], lj = fr[2 * (s / ps)], sj = fr[2 * (s / ps) + 1];
    float v[32];
    float* rowq = qs + idx * q;
    for (int i = 0; i < q; i++) {
        const float a = (rowq[i] - loc0) / scale0;
        const float b = a * sj;
        v[i] = b + lj;
    }
    clamp_nonfinite(v, q);
    for (int i = 0; i < q; i++) rowq[i] = v[i];
}

// Store a block's quantiles: steps [done, done + blen) of each row's forecast, those before the
// horizon (blockDecode :502-507). Rows r < R go to out, the mirrored rows to mir.
__global__ void ts_store_block(const float* qs, int rows, int batch, int vall, int V, int blen, int done, int horizon,
                               int q, float* out, float* mir) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * blen * q) return;
    const int i = (int)(idx % q);
    const int64_t rs = idx / q;
    const int r = (int)(rs / blen), s = (int)(rs % blen);
    const int g = r / vall, vi = r % vall;
    if (done + s >= horizon || vi >= V) return;
    const int64_t orow = (int64_t)(g < batch ? g : g - batch) * V + vi;
    float* dst = (g < batch ? out : mir) + (orow * horizon + done + s) * q;
    dst[i] = qs[idx];
}

// blockDecode's feedback (forecaster.zig:512-555) for target rows: the block's medians (0 when not
// finite or at least the extreme threshold) become observed steps [t, t + blen) of the context.
__global__ void ts_feedback(const float* qs, int rows, int vall, int V, int blen, int q, int median, float extreme,
                            float* ctx, uint8_t* mask, int cap_t, int t) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * blen) return;
    const int r = (int)(idx / blen), s = (int)(idx % blen);
    if (r % vall >= V) return;  // covariate rows: the window already holds their next steps
    float mv = qs[idx * q + median];
    if (!isfinite(mv) || fabsf(mv) >= extreme) mv = 0.f;
    ctx[(int64_t)r * cap_t + t + s] = mv;
    mask[(int64_t)r * cap_t + t + s] = 1;
}

// The context window after a drop of the oldest steps (forecaster.zig:514-530): dst[r, j] =
// src[r, start + j] for j < keep.
__global__ void ts_slide(const float* src, const uint8_t* src_mask, float* dst, uint8_t* dst_mask, int rows, int cap_t,
                         int start, int keep) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * keep) return;
    const int r = (int)(idx / keep), j = (int)(idx % keep);
    dst[(int64_t)r * cap_t + j] = src[(int64_t)r * cap_t + start + j];
    dst_mask[(int64_t)r * cap_t + j] = src_mask[(int64_t)r * cap_t + start + j];
}

// forecastRaw's quantile cap (forecaster.zig:396-418) bounds of each row from its original context:
// [min - a, max + a] over the observed values (0 when none), a = scale of the last patch x cap_k.
__global__ void ts_cap_bounds(const float* ctx, const uint8_t* mask, int cap_t, int t, int ps, const float* scale,
                              int cap_p, int rows, float cap_k, float* bounds) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float mx = -INFINITY, mn = INFINITY;
    for (int j = 0; j < t; j++)
        if (mask[(int64_t)r * cap_t + j]) {
            mx = fmaxf(mx, ctx[(int64_t)r * cap_t + j]);
            mn = fminf(mn, ctx[(int64_t)r * cap_t + j]);
        }
    if (isinf(mx)) mx = 0.f;
    if (isinf(mn)) mn = 0.f;
    const float a = scale[(int64_t)r * cap_p + t / ps - 1] * cap_k;
    bounds[2 * r] = mn - a;
    bounds[2 * r + 1] = mx + a;
}

// forecast's end (forecaster.zig:107-140, finish :163-178): each pass capped to its own bounds
// (std.math.clamp: @max(lo, @min(x, hi))), the mirrored pass averaged in level-reversed order, and
// series whose observed values are all non-negative clipped at 0.
__global__ void ts_final(float* out, const float* mir, const float* bounds, const uint8_t* nonneg, int R, int V,
                         int vall, int horizon, int q, int cap, int symmetric, int clip) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)R * horizon) return;
    const int r = (int)(idx / horizon);
    // bounds are per context row: target i of series s is row s * vall + i, its mirror R / V groups on
    const int fr = (r / V) * vall + r % V, mr = fr + (R / V) * vall;
    float* o = out + idx * q;
    float v[32];
    for (int j = 0; j < q; j++) {
        float f = o[j];
        if (cap) f = fmaxf(bounds[2 * fr], fminf(f, bounds[2 * fr + 1]));
        v[j] = f;
    }
    if (symmetric) {
        const float* m = mir + idx * q;
        for (int j = 0; j < q; j++) {
            float g = m[q - 1 - j];
            if (cap) g = fmaxf(bounds[2 * mr], fminf(g, bounds[2 * mr + 1]));
            const float s = v[j] + -g;
            v[j] = 0.5f * s;
        }
    }
    const bool cl = clip && nonneg[r];
    for (int j = 0; j < q; j++) o[j] = cl ? fmaxf(v[j], 0.f) : v[j];
}

unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

hipError_t launch_ts_stats(const TsStatsParams& p, hipStream_t s) {
    hipLaunchKernelGGL(ts_stats, dim3(blocks_for(p.rows, 64)), dim3(64), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_ts_features(const float* ctx, const uint8_t* mask, int cap_t, const float* loc, const float* scale,
                              int cap_p, int rows, int p0, int l, int ps, int use_asinh, const uint8_t* no_asinh,
                              float* feats, hipStream_t s) {
    const int64_t n = (int64_t)rows * (l - p0) * ps;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(ts_features, dim3(blocks_for(n, 256)), dim3(256), 0, s, ctx, mask, cap_t, loc, scale, cap_p, rows,
                       p0, l, ps, use_asinh, no_asinh, feats);
    return hipGetLastError();
}

hipError_t launch_ts_rope_tables(const int* row_first, int groups, int vall, int n_tok, int ne, int shift,
                                 const TsRope& rp, float* cos_t, float* sin_t, int* first_obs, hipStream_t s) {
    hipLaunchKernelGGL(ts_rope_tables, dim3(blocks_for((int64_t)n_tok * 32, 256), (unsigned)groups), dim3(256), 0, s,
                       row_first, vall, n_tok, ne, shift, rp, cos_t, sin_t, first_obs);
    return hipGetLastError();
}

hipError_t launch_ts_assemble(const float* emb, const float* query, float* x, int rows, int m, int h, int d,
                              hipStream_t s) {
    hipLaunchKernelGGL(ts_assemble, dim3(blocks_for((int64_t)rows * (m + h) * (d / 4), 256)), dim3(256), 0, s, emb,
                       query, x, rows, m, h, d);
    return hipGetLastError();
}

hipError_t launch_ts_mul_sigmoid(float* o, const float* g, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(ts_mul_sigmoid, dim3(blocks_for(n / 4, 256)), dim3(256), 0, s, o, g, n / 4);
    return hipGetLastError();
}

hipError_t launch_ts_from_bf16(const uint16_t* oh, const float* g, float* o, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(ts_from_bf16, dim3(blocks_for(n / 4, 256)), dim3(256), 0, s, oh, g, o, n / 4);
    return hipGetLastError();
}

hipError_t launch_ts_mul_silu(const float* hbuf, float* a, int64_t tokens, int hid, hipStream_t s) {
    hipLaunchKernelGGL(ts_mul_silu, dim3(blocks_for(tokens * (hid / 4), 256)), dim3(256), 0, s, hbuf, a, tokens, hid);
    return hipGetLastError();
}

hipError_t launch_ts_head_finish(const float* raw, const float* loc, const float* scale, int cap_p, int l, int rows,
                                 int h, const TsHead& hp, float* qs, hipStream_t s) {
    hipLaunchKernelGGL(ts_head_finish, dim3(blocks_for((int64_t)rows * h * hp.ps, 128)), dim3(128), 0, s, raw, loc,
                       scale, cap_p, l, rows, h, hp, qs);
    return hipGetLastError();
}

hipError_t launch_ts_refine(float* qs, const float* loc, const float* scale, int cap_p, int l, const double* fold,
                            int rows, int h, int ps, int q, int median, double min_scale, float* frames,
                            hipStream_t s) {
    hipLaunchKernelGGL(ts_refine_frames, dim3(blocks_for(rows, 64)), dim3(64), 0, s, qs, loc, scale, cap_p, l, fold, rows,
                       h, ps, q, median, min_scale, frames);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(ts_refine_apply, dim3(blocks_for((int64_t)rows * h * ps, 128)), dim3(128), 0, s, qs, frames, rows,
                       h, ps, q);
    return hipGetLastError();
}

hipError_t launch_ts_store_block(const float* qs, int rows, int batch, int vall, int V, int blen, int done, int horizon,
                                 int q, float* out, float* mir, hipStream_t s) {
    hipLaunchKernelGGL(ts_store_block, dim3(blocks_for((int64_t)rows * blen * q, 256)), dim3(256), 0, s, qs, rows,
                       batch, vall, V, blen, done, horizon, q, out, mir);
    return hipGetLastError();
}

hipError_t launch_ts_feedback(const float* qs, int rows, int vall, int V, int blen, int q, int median, float extreme,
                              float* ctx, uint8_t* mask, int cap_t, int t, hipStream_t s) {
    hipLaunchKernelGGL(ts_feedback, dim3(blocks_for((int64_t)rows * blen, 256)), dim3(256), 0, s, qs, rows, vall, V,
                       blen, q, median, extreme, ctx, mask, cap_t, t);
    return hipGetLastError();
}

hipError_t launch_ts_slide(const float* src, const uint8_t* src_mask, float* dst, uint8_t* dst_mask, int rows,
                           int cap_t, int start, int keep, hipStream_t s) {
    hipLaunchKernelGGL(ts_slide, dim3(blocks_for((int64_t)rows * keep, 256)), dim3(256), 0, s, src, src_mask, dst,
                       dst_mask, rows, cap_t, start, keep);
    return hipGetLastError();
}

hipError_t launch_ts_cap_bounds(const float* ctx, const uint8_t* mask, int cap_t, int t, int ps, const float* scale,
                                int cap_p, int rows, float cap_k, float* bounds, hipStream_t s) {
    hipLaunchKernelGGL(ts_cap_bounds, dim3(blocks_for(rows, 64)), dim3(64), 0, s, ctx, mask, cap_t, t, ps, scale, cap_p,
                       rows, cap_k, bounds);
    return hipGetLastError();
}

hipError_t launch_ts_final(float* out, const float* mir, const float* bounds, const uint8_t* nonneg, int R, int V,
                           int vall, int horizon, int q, int cap, int symmetric, int clip, hipStream_t s) {
    hipLaunchKernelGGL(ts_final, dim3(blocks_for((int64_t)R * horizon, 128)), dim3(128), 0, s, out, mir, bounds, nonneg,
                       R, V, vall, horizon, q, cap, symmetric, clip);
    return hipGetLastError();
}

}  // namespace tsfm
