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
    for (int i = 4 * lane; i < dim; i += 256) {
        const f32x4 v = ld4(xr + i);
        ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    float* o = out + (int64_t)row * out_tok;
    for (int i = 4 * lane; i < dim; i += 256) {
#pragma clang fp contract(off)
        const f32x4 t = ld4(xr + i) * inv;  // x * inv * scale, left to right like the Zig
        st4(o + i, t * ld4(scale + i));
    }
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

// The Chronos-Bolt forecaster's per-series preparation (src/chronos_bolt/forecaster.zig:150-196),
// one workgroup per series: the instance norm over the observed (non-NaN) values, with the sums
// in double as the Zig does (count, sum, then sum of (x - loc)^2 with x - loc in f32; a zero scale
// becomes norm_eps), then the [values, mask] features of n_patch patches left-padded with pad
// missing steps, and each patch's "has an observation" byte.
__global__ __launch_bounds__(256) void bolt_prepare(const float* ctx, int64_t stride, int64_t offset, int len,
                                                    int ps, int n_patch, int pad, float norm_eps, float* feats,
                                                    uint8_t* patch_valid, float* loc, float* scale) {
    __shared__ double red[256];
    const int li = blockIdx.x, tid = threadIdx.x;
    const float* row = ctx + (int64_t)li * stride + offset;
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
    float lo = 0.f, sc = 1.f;
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
