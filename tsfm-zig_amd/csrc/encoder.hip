// Row normalisation for the encoder stack (gfx950): nn.rmsNorm (src/core/nn.zig:361-396).
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

}  // namespace

hipError_t launch_rms_norm(const float* x, int64_t x_tok, float* out, int64_t out_tok, const float* scale, int rows,
                           int dim, float eps, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (dim <= 0 || dim % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rms_norm_rows, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, x, x_tok, out, out_tok,
                       scale, rows, dim, eps);
    return hipGetLastError();
}

}  // namespace tsfm
