// Chronos-Bolt horizons longer than one block (gfx950): the block store, the context window of the
// quantile paths, and the empirical quantiles of the q x q samples per step.
//
// Reference: src/chronos_bolt/forecaster.zig forecast (:22-78), quantileLinear (:81-92),
// storeBlock (:95-103).
#include "common.hpp"
#include "launch.hpp"

#pragma clang fp contract(off)

namespace tsfm {
namespace {

// storeBlock: out[(s * horizon + start + p) * q + qi] = pred[(s * q + qi) * P + p] for the steps
// before the horizon.
__global__ __launch_bounds__(256) void bolt_store_block(const float* pred, int b, int q, int P, int horizon, int start,
                                                        float* out) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)b * P * q) return;
    const int qi = (int)(idx % q);
    const int64_t sp = idx / q;
    const int s = (int)(sp / P), p = (int)(sp % P);
    if (start + p >= horizon) return;
    out[((int64_t)s * horizon + start + p) * q + qi] = pred[((int64_t)s * q + qi) * P + p];
}

// The next window of each quantile path (forecaster.zig:51-60): step i of the new row is step
// skip + i of (old row ++ the path's block), skip = len + P - new_len.
__global__ __launch_bounds__(256) void bolt_window(const float* src, int64_t src_stride, int64_t src_off, int len,
                                                   int rep, const float* pred, int P, float* dst, int new_len,
                                                   int rows) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)rows * new_len) return;
    const int r = (int)(idx / new_len), i = (int)(idx % new_len);
    const int j = len + P - new_len + i;
    dst[idx] = j < len ? src[(int64_t)(r / rep) * src_stride + src_off + j] : pred[(int64_t)r * P + (j - len)];
}

// quantileLinear: torch.quantile's linear interpolation of an ascending slice, with ATen's lerp
// (from the low end when the weight is below 0.5, else from the high end).
__device__ float quantile_linear(const float* a, int n, float level) {
    const float rank = level * (float)(n - 1);
    const float lo_f = floorf(rank);
    const int lo = (int)lo_f, hi = min((int)ceilf(rank), n - 1);
    const float w = rank - lo_f, x = a[lo], y = a[hi];
    return w < 0.5f ? x + w * (y - x) : y - (y - x) * (1.f - w);
}

// One thread per (series, step): the q * q samples raw[(s q q + k) P + p] sorted ascending in the
// thread's LDS slice (insertion sort), then the q levels.
__global__ __launch_bounds__(64) void bolt_sample_quantiles(const float* raw, int b, int q, int P, BoltLevels lv,
                                                            float* pred) {
    extern __shared__ float lds[];
    const int n = q * q;
    const int64_t idx = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (idx >= (int64_t)b * P) return;
    const int s = (int)(idx / P), p = (int)(idx % P);
    float* a = lds + threadIdx.x * n;
    for (int k = 0; k < n; k++) {
        const float v = raw[((int64_t)s * n + k) * P + p];
        int j = k;
        while (j > 0 && v < a[j - 1]) {
            a[j] = a[j - 1];
            j--;
        }
        a[j] = v;
    }
    for (int qi = 0; qi < q; qi++) pred[((int64_t)s * q + qi) * P + p] = quantile_linear(a, n, lv.v[qi]);
}

unsigned blocks(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

hipError_t launch_bolt_store_block(const float* pred, int b, int q, int P, int horizon, int start, float* out,
                                   hipStream_t s) {
    hipLaunchKernelGGL(bolt_store_block, dim3(blocks((int64_t)b * P * q, 256)), dim3(256), 0, s, pred, b, q, P, horizon,
                       start, out);
    return hipGetLastError();
}

hipError_t launch_bolt_window(const float* src, int64_t src_stride, int64_t src_off, int len, int rep,
                              const float* pred, int P, float* dst, int new_len, int rows, hipStream_t s) {
    hipLaunchKernelGGL(bolt_window, dim3(blocks((int64_t)rows * new_len, 256)), dim3(256), 0, s, src, src_stride,
                       src_off, len, rep, pred, P, dst, new_len, rows);
    return hipGetLastError();
}

hipError_t launch_bolt_sample_quantiles(const float* raw, int b, int q, int P, const BoltLevels& lv, float* pred,
                                        hipStream_t s) {
    if (q < 1 || q > 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(bolt_sample_quantiles, dim3(blocks((int64_t)b * P, 64)), dim3(64), (size_t)64 * q * q * 4, s, raw,
                       b, q, P, lv, pred);
    return hipGetLastError();
}

}  // namespace tsfm
