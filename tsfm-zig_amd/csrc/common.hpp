// Shared device-side definitions for the tsfm attention kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace tsfm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));  // not HIP's float2: a union-based struct
                                                          // that the optimiser cannot keep in registers
                                                          // once it sits inside another struct

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Two floats rounded to bf16 (BF16) or f16, round to nearest even, packed low-first.
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (BF16) {
        const bf16x2 v = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        const f16x2 v = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
}

constexpr int kHeadDim = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();
constexpr float kFltMax = 3.40282347e+38f;

// Mask values: attn.Mask declaration order (src/core/attn.zig:10-21) plus the Timestral decoder
// rows (src/timestral/model.zig:612-632). Same numbering as TSFM_MASK_* in tsfm_attn.h.
enum Mask : int { FULL = 0, KEYS_ADDITIVE = 1, CAUSAL = 2, CAUSAL_KEYS = 3, FULL_KEYS = 4, DECODER = 5 };
enum BiasKind : int { BIAS_NONE = 0, BIAS_DENSE = 1, BIAS_REL = 2 };

// Longest T5 relative-offset table kept in LDS (n_q + n_k - 1 entries).
constexpr int kRelMax = 2048;

// Kernel arguments, by value. Strides are in elements.
struct Params {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    int64_t q_tok, q_batch, k_tok, k_batch, v_tok, v_batch, o_tok, o_batch;
    const uint8_t* key_valid;
    int64_t kv_batch;
    const float* bias;
    int64_t bias_head, bias_row;
    const float* rel_table;
    const int32_t* rel_bucket;
    int32_t rel_buckets;
    const float* rope_cos;
    const float* rope_sin;
    int64_t rope_table_stride;
    int32_t rope_rows_per_table, rope_row0;
    int32_t B, H, n_q, n_k, q_pos0, ctx_keys, chain_start;
    float scale;
};

// Workgroup ids are dealt round-robin over the 8 XCDs (id % 8). Re-map them so that consecutive
// logical ids -- the query tiles of one (series, head), which read the same K/V -- run on the
// same XCD and share its L2. A bijection on [0, n) for any n.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
    const int xcd = bid & 7, idx = bid >> 3, full = n >> 3, rem = n & 7;
    return xcd < rem ? xcd * (full + 1) + idx : rem * (full + 1) + (xcd - rem) * full + idx;
}

// Key index range a query at position qpos may read under each mask, and the exclusive end of
// keys any query of [qpos_lo, qpos_hi] may read (used to skip whole tiles).
template <int MASK>
__device__ __forceinline__ int key_end_for(int qpos_hi, int n_k, int ctx_keys) {
    if (MASK == CAUSAL || MASK == CAUSAL_KEYS) return min(n_k, qpos_hi + 1);
    if (MASK == DECODER) return min(n_k, max(ctx_keys, qpos_hi + 1));
    return n_k;
}

// One score after scale and bias: the reference's mask rule (src/core/attn.zig:35-67,
// src/timestral/model.zig:612-632). Keys past n_k are tile padding and always excluded.
template <int MASK>
__device__ __forceinline__ float apply_mask(float x, int key, int qpos, int n_k, bool valid, int ctx_keys,
                                            int chain_start) {
    if (key >= n_k) return kNegInf;
    if (MASK == KEYS_ADDITIVE) return valid ? x : x + (-kFltMax);
    if (MASK == CAUSAL) return key <= qpos ? x : kNegInf;
    if (MASK == CAUSAL_KEYS) return (key == qpos || (valid && key <= qpos)) ? x : kNegInf;
    if (MASK == FULL_KEYS) return (key == qpos || valid) ? x : kNegInf;
    if (MASK == DECODER) return ((key < ctx_keys && valid) || (key >= chain_start && key <= qpos)) ? x : kNegInf;
    return x;
}

// Additive mask term of one key: the part of the reference's mask rule (src/core/attn.zig:35-67,
// src/timestral/model.zig:612-632) that depends on the key alone. Keys past n_k are tile padding.
template <int MASK>
__device__ __forceinline__ float key_term(int key, int n_k, bool valid, int ctx_keys) {
    if (key >= n_k) return kNegInf;
    if (MASK == KEYS_ADDITIVE) return valid ? 0.f : -kFltMax;
    if (MASK == CAUSAL_KEYS || MASK == FULL_KEYS) return valid ? 0.f : kNegInf;
    if (MASK == DECODER) return (key < ctx_keys && valid) ? 0.f : kNegInf;
    return 0.f;  // FULL, CAUSAL
}

// The whole mask rule for one scaled, biased score x, given its key term ka.
template <int MASK>
__device__ __forceinline__ float masked(float x, float ka, int key, int qpos, int n_k, int chain_start) {
    if (MASK == CAUSAL) return key <= qpos ? x + ka : kNegInf;
    if (MASK == CAUSAL_KEYS) return (key == qpos && key < n_k) ? x : (key <= qpos ? x + ka : kNegInf);
    if (MASK == FULL_KEYS) return (key == qpos && key < n_k) ? x : x + ka;
    if (MASK == DECODER) return (key >= chain_start && key <= qpos && key < n_k) ? x : x + ka;
    return x + ka;  // FULL, KEYS_ADDITIVE: x + 0, x + (-FLT_MAX), or -inf for padding
}

// Bytes of key_valid per row the mask reads: DECODER only tests keys below ctx_keys.
template <int MASK>
__device__ __forceinline__ int valid_len(int n_k, int ctx_keys) {
    return MASK == DECODER ? min(n_k, ctx_keys) : n_k;
}

template <int MASK>
constexpr bool mask_reads_valid() {
    return MASK == KEYS_ADDITIVE || MASK == CAUSAL_KEYS || MASK == FULL_KEYS || MASK == DECODER;
}

// Rotate-half RoPE of four pairs (nn.ropeHalf, src/core/nn.zig:453-460): lo holds dims i..i+3,
// hi dims i+half..i+half+3. Unfused products, like the Zig code.
__device__ __forceinline__ void rope4(f32x4& lo, f32x4& hi, f32x4 c, f32x4 s) {
#pragma clang fp contract(off)
    const f32x4 x1 = lo, x2 = hi;
    lo = x1 * c - x2 * s;
    hi = x2 * c + x1 * s;
}

constexpr int kLutPad = 32;  // T5 table margin on each side (entries): one 32-key chunk

// T5 bias of head h by relative index t = j - i + n_q - 1, stored at lut_raw[kLutPad + t] for t in
// [-kLutPad, n_q + n_k - 1 + kLutPad): the margins repeat the end values (the bucket of the nearest
// real index), so padded keys and query slots index it without a clamp.
__device__ __forceinline__ void fill_rel_lut(float* lut_raw, const Params& p, int h, int tid, int nthreads) {
    const int n_rel = p.n_q + p.n_k - 1;
    for (int u = tid; u < n_rel + 2 * kLutPad; u += nthreads) {
        const int t = min(max(u - kLutPad, 0), n_rel - 1);
        lut_raw[u] = p.rel_table[min(max(p.rel_bucket[t], 0), p.rel_buckets - 1) * p.H + h];
    }
}

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x2 ld2(const float* p) { return *reinterpret_cast<const f32x2*>(p); }
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
__device__ __forceinline__ void st2(float* p, f32x2 v) { *reinterpret_cast<f32x2*>(p) = v; }

// Rotate-half RoPE of two pairs, as rope4.
__device__ __forceinline__ void rope2(f32x2& lo, f32x2& hi, f32x2 c, f32x2 s) {
#pragma clang fp contract(off)
    const f32x2 x1 = lo, x2 = hi;
    lo = x1 * c - x2 * s;
    hi = x2 * c + x1 * s;
}

// Word 3 of a raw buffer descriptor on gfx9 parts: 32-bit data format, no swizzle. Loads past the
// descriptor's byte count return 0.
constexpr int kBufferConfig = 0x00020000;

// Raw buffer over `bytes` bytes at base, and loads at a per-lane byte offset: a 32-bit offset in
// one VGPR instead of a 64-bit pointer in two, and zeros instead of a fault past the end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buf(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferConfig);
}
// 16 bytes per lane from a buffer straight into LDS (lane l's at lds + 16 l), issued as inline
// assembly: the compiler then does not see an LDS write whose address it cannot separate from the
// kernel's LDS reads, and does not put a wait for every outstanding global load in front of them.
// A caller reads what a load fills only after its own `s_waitcnt vmcnt(0)` and a barrier.
// (Loads the compiler does not know of only make its own vmcnt waits more conservative.)
// lds and soff are wave-uniform (taken from the first lane, so they sit in SGPRs).
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(rsrc),
                   "s"(__builtin_amdgcn_readfirstlane(soff))
                 : "memory", "m0");
}
// Raw buffer descriptor over `bytes` bytes at base (loads past the end return 0), in SGPRs.
__device__ __forceinline__ u32x4 buf_desc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                 (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu)),
                 (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes), (uint32_t)kBufferConfig};
}
__device__ __forceinline__ float bld1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ f32x2 bld2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ f32x4 bld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Max / sum over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48), on the VALU with
// gfx950's lane swaps: permlane32_swap(x, x) returns (x of lanes 0-31 in both halves, x of lanes
// 32-63 in both halves), permlane16_swap likewise for even/odd 16-lane rows. Every lane ends with
// the same value, combined in the same order.
__device__ __forceinline__ float max4(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum4(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// nn.rmsNorm pieces shared by every kernel that normalises a row (one wave per row, lane l
// holding the four-column groups 4 l, 4 l + 256, ...): the lane's running sum of squares, the
// wave-wide total, and the scaled output x * inv * scale, left to right.
// Products and sums stay unfused (as the reference's vector `acc += v * v`), so every kernel that
// shares these helpers rounds the same way.
__device__ inline float sumsq4(float ss, f32x4 v) {
#pragma clang fp contract(off)
    return ss + (v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3]);
}

__device__ inline float rms_inv(float ss, int dim, float eps) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    return 1.0f / sqrtf(ss / (float)dim + eps);
}

__device__ inline f32x4 rms_apply(f32x4 x, float inv, f32x4 scale) {
#pragma clang fp contract(off)
    const f32x4 t = x * inv;
    return t * scale;
}

}  // namespace tsfm
