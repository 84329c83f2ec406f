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

}  // namespace

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
