// Row kernels around the Chronos-2 encoder stack (gfx950): nn.rmsNorm (src/core/nn.zig:361-396),
// and the forecaster's sequence assembly and future-token gather.
//
// out[r, :] = x[r, :] * (1 / sqrt(mean(x[r, :]^2) + eps)) * scale, one wave per row: each lane
// takes 16-byte groups 4 lane, 4 lane + 256, ...; the sum of squares is reduced across the wave,
// then the same lanes scale and store their groups. out may be x (every element is read before the
// row's reduction completes and written after it, by the same lane). HBM-bound: one read and one
// write of the row.
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

__global__ __launch_bounds__(256) void rms_norm_rows(const float* x, int64_t x_tok, float* out, int64_t out_tok,
                                                     const float* scale, int rows, int dim, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (int64_t)row * x_tok;
    float ss = 0.f;
    for (int i = 4 * lane; i < dim; i += 256) ss = sumsq4(ss, ld4(xr + i));
    const float inv = rms_inv(ss, dim, eps);
    float* o = out + (int64_t)row * out_tok;
    for (int i = 4 * lane; i < dim; i += 256) st4(o + i, rms_apply(ld4(xr + i), inv, ld4(scale + i)));
}

// Chronos-2 token sequence (src/chronos2/forecaster.zig:162-173): row li * seq + t of x is context
// embedding li * n_ctx + t for t < n_ctx, the [REG] token for t = n_ctx, and future embedding
// li * n_out + t - n_ctx - 1 after it; the key is valid when its context patch has an observation,
// and always for [REG] and the future patches. One wave per row.
__global__ __launch_bounds__(256) void assemble_sequence(const float* ctx_emb, const float* fut_emb, const float* reg,
                                                         const uint8_t* ctx_valid, float* x, uint8_t* key_valid,
                                                         int nb, int n_ctx, int n_out, int d) {
    const int seq = n_ctx + 1 + n_out;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= nb * seq) return;
    const int li = row / seq, t = row - li * seq;
    const float* src = t < n_ctx ? ctx_emb + ((int64_t)li * n_ctx + t) * d
                       : t == n_ctx ? reg
                                    : fut_emb + ((int64_t)li * n_out + (t - n_ctx - 1)) * d;
    float* dst = x + (int64_t)row * d;
    for (int i = 4 * lane; i < d; i += 256) st4(dst + i, ld4(src + i));
    if (lane == 0) key_valid[row] = t < n_ctx ? (ctx_valid[(int64_t)li * n_ctx + t] != 0) : 1;
}

// The future tokens' hidden states (src/chronos2/forecaster.zig:177-181): row li * n_out + p of
// hidden is row li * seq + n_ctx + 1 + p of x.
__global__ __launch_bounds__(256) void gather_future(const float* x, float* hidden, int nb, int n_ctx, int n_out,
                                                     int d) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= nb * n_out) return;
    const int li = row / n_out, pp = row - li * n_out;
    const float* src = x + ((int64_t)li * (n_ctx + 1 + n_out) + n_ctx + 1 + pp) * d;
    float* dst = hidden + (int64_t)row * d;
    for (int i = 4 * lane; i < d; i += 256) st4(dst + i, ld4(src + i));
}

// Every row of y is the same vector (the decoder start token, src/chronos_bolt/model.zig:281-282).
__global__ __launch_bounds__(256) void broadcast_rows(const float* v, float* y, int rows, int d) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    for (int i = 4 * lane; i < d; i += 256) st4(y + (int64_t)row * d + i, ld4(v + i));
}

// Fixed-order sum of one double per thread over a 256-thread workgroup (tree in LDS).
__device__ double block_sum(double v, double* red) {
    red[threadIdx.x] = v;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

// The forecasters' instance norm over one series' observed (non-NaN) values
// (src/chronos_bolt/forecaster.zig:153-172, src/chronos2/forecaster.zig:97-116), for a whole
// 256-thread workgroup: count, sum and then the sum of (x - loc)^2 with x - loc in f32 are kept
// in double as the Zig does; loc = f32(sum / count), scale = f32(sqrt(ss / count)), and a zero
// scale becomes norm_eps. No observation: loc 0, scale 1.
__device__ void instance_norm(const float* row, int len, float norm_eps, double* red, float& lo, float& sc) {
    const int tid = threadIdx.x;
    double cnt = 0.0, sum = 0.0;
    for (int i = tid; i < len; i += 256) {
        const float x = row[i];
        if (!__builtin_isnan(x)) {
            cnt += 1.0;
            sum += (double)x;
        }
    }
    cnt = block_sum(cnt, red);
    sum = block_sum(sum, red);
    lo = 0.f;
    sc = 1.f;
    if (cnt > 0.0) {
        lo = (float)(sum / cnt);
        double ss = 0.0;
        for (int i = tid; i < len; i += 256) {
            const float x = row[i];
            if (!__builtin_isnan(x)) {
                const float dv = x - lo;
                ss += (double)dv * (double)dv;
            }
        }
        ss = block_sum(ss, red);
        sc = (float)__builtin_sqrt(ss / cnt);
        if (sc == 0.f) sc = norm_eps;
    }
}

// The Chronos-Bolt forecaster's per-series preparation (src/chronos_bolt/forecaster.zig:150-196),
// one workgroup per series: the instance norm, then the [values, mask] features of n_patch
// patches left-padded with pad missing steps, and each patch's "has an observation" byte.
__global__ __launch_bounds__(256) void bolt_prepare(const float* ctx, int64_t stride, int64_t offset, int len,
                                                    int ps, int n_patch, int pad, float norm_eps, float* feats,
                                                    uint8_t* patch_valid, float* loc, float* scale) {
    __shared__ double red[256];
    const int li = blockIdx.x, tid = threadIdx.x;
    const float* row = ctx + (int64_t)li * stride + offset;
    float lo, sc;
    instance_norm(row, len, norm_eps, red, lo, sc);
    for (int e = tid; e < n_patch * ps; e += 256) {
        const int pp = e / ps, i = e - pp * ps;
        const int src = pp * ps + i - pad;
        float val = 0.f, obs = 0.f;
        if (src >= 0) {
            const float x = row[src];
            if (!__builtin_isnan(x)) {
                obs = 1.f;
                val = (x - lo) / sc;
            }
        }
        float* f = feats + ((int64_t)li * n_patch + pp) * 2 * ps;
        f[i] = val;
        f[ps + i] = obs;
    }
    for (int pp = tid; pp < n_patch; pp += 256) {
        bool any = false;
        for (int i = 0; i < ps; i++) {
            const int src = pp * ps + i - pad;
            any = any || (src >= 0 && !__builtin_isnan(row[src]));
        }
        patch_valid[(int64_t)li * n_patch + pp] = any ? 1 : 0;
    }
    if (tid == 0) {
        loc[li] = lo;
        scale[li] = sc;
    }
}

// The Chronos-2 forecaster's per-series preparation (src/chronos2/forecaster.zig:93-153), one
// workgroup per series: the instance norm (zero scale -> 1e-5), then the [time_enc, values, mask]
// features of n_ctx context patches (left-padded with pad missing steps; values optionally
// asinh'd) with their "has an observation" byte, and of n_out future patches, which carry only
// their time encoding. Time encodings are (j - n_ctx * ps) / tscale and j / tscale in f32.
__global__ __launch_bounds__(256) void chronos2_prepare(const float* inputs, int64_t stride, int64_t start, int len,
                                                        int ps, int n_ctx, int n_out, int pad, float tscale,
                                                        int arcsinh, float* feats, float* fut_feats,
                                                        uint8_t* ctx_valid, float* loc, float* scale) {
    __shared__ double red[256];
    const int li = blockIdx.x, tid = threadIdx.x;
    const float* row = inputs + (int64_t)li * stride + start;
    float lo, sc;
    instance_norm(row, len, 1e-5f, red, lo, sc);
    const float origin = (float)(n_ctx * ps);
    for (int e = tid; e < n_ctx * ps; e += 256) {
        const int pp = e / ps, i = e - pp * ps;
        const int src = e - pad;
        float val = 0.f, obs = 0.f;
        if (src >= 0 && src < len) {
            const float x = row[src];
            if (!__builtin_isnan(x)) {
                obs = 1.f;
                val = (x - lo) / sc;
                if (arcsinh) val = asinhf(val);
            }
        }
        float* f = feats + ((int64_t)li * n_ctx + pp) * 3 * ps;
        f[i] = ((float)e - origin) / tscale;
        f[ps + i] = val;
        f[2 * ps + i] = obs;
    }
    for (int pp = tid; pp < n_ctx; pp += 256) {
        bool any = false;
        for (int i = 0; i < ps; i++) {
            const int src = pp * ps + i - pad;
            any = any || (src >= 0 && src < len && !__builtin_isnan(row[src]));
        }
        ctx_valid[(int64_t)li * n_ctx + pp] = any ? 1 : 0;
    }
    for (int e = tid; e < n_out * ps; e += 256) {
        const int pp = e / ps, i = e - pp * ps;
        float* f = fut_feats + ((int64_t)li * n_out + pp) * 3 * ps;
        f[i] = (float)e / tscale;
        f[ps + i] = 0.f;
        f[2 * ps + i] = 0.f;
    }
    if (tid == 0) {
        loc[li] = lo;
        scale[li] = sc;
    }
}

// The Chronos-2 inverse scaling (src/chronos2/forecaster.zig:184-201): out (n, horizon, q) from
// raw (n * n_out, q * ps), where step p * ps + i of quantile qi is raw[(li * n_out + p) * q * ps
// + qi * ps + i]; sinh first when the model works in asinh space, then v * scale + loc unfused.
__global__ __launch_bounds__(256) void chronos2_finish(const float* raw, const float* loc, const float* scale,
                                                       float* out, int n, int n_out, int q, int ps, int horizon,
                                                       int arcsinh) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per = (int64_t)horizon * q;
    if (idx >= (int64_t)n * per) return;
    const int li = (int)(idx / per);
    const int rem = (int)(idx - li * per), step = rem / q, qi = rem - step * q;
    const int pp = step / ps, i = step - pp * ps;
    float v = raw[((int64_t)li * n_out + pp) * q * ps + qi * ps + i];
    if (arcsinh) v = sinhf(v);
    {
#pragma clang fp contract(off)
        out[idx] = v * scale[li] + loc[li];
    }
}

// The inverse instance norm (src/chronos_bolt/forecaster.zig:215-219): out = raw * scale + loc.
__global__ __launch_bounds__(256) void bolt_finish(const float* raw, const float* loc, const float* scale, float* out,
                                                   int n, int per) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)n * per) return;
    const int li = (int)(idx / per);
    {
#pragma clang fp contract(off)
        out[idx] = raw[idx] * scale[li] + loc[li];  // unfused, like the Zig
    }
}

}  // namespace

hipError_t launch_bolt_prepare(const float* ctx, int64_t stride, int64_t offset, int len, int ps, int n_patch, int pad,
                               float norm_eps, float* feats, uint8_t* patch_valid, float* loc, float* scale, int n,
                               hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(bolt_prepare, dim3((unsigned)n), dim3(256), 0, stream, ctx, stride, offset, len, ps, n_patch, pad,
                       norm_eps, feats, patch_valid, loc, scale);
    return hipGetLastError();
}

hipError_t launch_chronos2_prepare(const float* inputs, int64_t stride, int64_t start, int len, int ps, int n_ctx,
                                  int n_out, int pad, float tscale, int arcsinh, float* feats, float* fut_feats,
                                  uint8_t* ctx_valid, float* loc, float* scale, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(chronos2_prepare, dim3((unsigned)n), dim3(256), 0, stream, inputs, stride, start, len, ps, n_ctx,
                       n_out, pad, tscale, arcsinh, feats, fut_feats, ctx_valid, loc, scale);
    return hipGetLastError();
}

hipError_t launch_chronos2_finish(const float* raw, const float* loc, const float* scale, float* out, int n, int n_out,
                                  int q, int ps, int horizon, int arcsinh, hipStream_t stream) {
    const int64_t total = (int64_t)n * horizon * q;
    if (total <= 0) return hipSuccess;
    if (horizon > n_out * ps) return hipErrorInvalidValue;
    hipLaunchKernelGGL(chronos2_finish, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, raw, loc, scale,
                       out, n, n_out, q, ps, horizon, arcsinh);
    return hipGetLastError();
}

hipError_t launch_bolt_finish(const float* raw, const float* loc, const float* scale, float* out, int n, int per,
                              hipStream_t stream) {
    const int64_t total = (int64_t)n * per;
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(bolt_finish, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, raw, loc, scale, out, n,
                       per);
    return hipGetLastError();
}

hipError_t launch_broadcast_rows(const float* v, float* y, int rows, int d, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (d % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(broadcast_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, v, y, rows, d);
    return hipGetLastError();
}

hipError_t launch_assemble_sequence(const float* ctx_emb, const float* fut_emb, const float* reg,
                                    const uint8_t* ctx_valid, float* x, uint8_t* key_valid, int nb, int n_ctx,
                                    int n_out, int d, hipStream_t stream) {
    const int64_t rows = (int64_t)nb * (n_ctx + 1 + n_out);
    if (rows <= 0) return hipSuccess;
    if (d % 4 || rows > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(assemble_sequence, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, ctx_emb, fut_emb,
                       reg, ctx_valid, x, key_valid, nb, n_ctx, n_out, d);
    return hipGetLastError();
}

hipError_t launch_gather_future(const float* x, float* hidden, int nb, int n_ctx, int n_out, int d,
                                hipStream_t stream) {
    const int64_t rows = (int64_t)nb * n_out;
    if (rows <= 0) return hipSuccess;
    if (d % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gather_future, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, hidden, nb, n_ctx,
                       n_out, d);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float* x, int64_t x_tok, float* out, int64_t out_tok, const float* scale, int rows,
                           int dim, float eps, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (dim <= 0 || dim % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rms_norm_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, x_tok, out, out_tok,
                       scale, rows, dim, eps);
    return hipGetLastError();
}

}  // namespace tsfm
