// Fused f32 attention for gfx950: one workgroup = one (series, head) x 128 queries.
//
// The reference computes one (series, head) at a time with a materialised n x n score matrix:
// gemmNT -> bias -> masked softmax -> gemmNN (src/core/attn.zig:72-96). Here the whole batch is one
// launch and no score matrix exists: K/V tiles of 64 keys are staged in LDS and both products run
// on the f32 matrix cores (v_mfma_f32_16x16x4_f32) with an online softmax in registers.
//
// Wave layout (4 waves x 32 queries):
//   S^T = K . Q^T   A = K tile rows (16 keys) from LDS, B = Q^T (16 queries) held in VGPRs.
//                   Accumulator lane l holds query l%16 and keys 4*(l/16)+r, r=0..3.
//   O^T += V^T . P^T  A = V^T (16 dims x 4 keys) from LDS, B = P^T straight from the S^T
//                   accumulator: register r of lane l is key 4*(l/16)+r, exactly the k-slot the
//                   instruction expects, so P never leaves registers.
//   O^T accumulator lane l holds query l%16 and dims 4*(l/16)+r: the same query as the softmax
//   state of that lane, so the online rescale is a plain multiply.
// The contraction order over head dims is permuted (lane group g holds dims 8g..8g+7 and
// 32+8g..32+8g+7) so that every RoPE pair (i, i+32) sits in one lane and K reads are 128-bit.
//
// LDS: K tile [64 keys][68] (padded: conflict-free 128-bit reads), V tile [16 key quads][64][4]
// (transposed so one 128-bit read gives the four keys of one MFMA group), key mask, T5 bias LUT.
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

constexpr int NK = 64;       // keys per LDS tile
constexpr int QW = 32;       // queries per wave (2 blocks of 16)
constexpr int NWAVE = 4;
constexpr int QT = QW * NWAVE;  // queries per workgroup
constexpr int KPAD = 68;     // K row pitch in LDS (floats)

template <int MASK, int BIAS, bool ROPE>
__global__ __launch_bounds__(256) void attn_fwd_f32(Params p) {
    __shared__ __attribute__((aligned(16))) float Ks[NK * KPAD];
    __shared__ __attribute__((aligned(16))) float Vs[NK * kHeadDim];
    __shared__ __attribute__((aligned(16))) uint8_t kvs[NK];
    __shared__ float lut[BIAS == BIAS_REL ? kRelMax : 1];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ql = lane & 15, g = lane >> 4;
    const int q_tiles = (p.n_q + QT - 1) / QT;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = logical / q_tiles;
    int qt = logical % q_tiles;
    if (MASK == CAUSAL || MASK == CAUSAL_KEYS) qt = q_tiles - 1 - qt;  // longest rows first
    const int b = bh / p.H, h = bh % p.H;
    const int q0 = qt * QT;
    const int wq0 = q0 + wave * QW;

    const float* __restrict__ Q = static_cast<const float*>(p.q) + b * p.q_batch + h * kHeadDim;
    const float* __restrict__ K = static_cast<const float*>(p.k) + b * p.k_batch + h * kHeadDim;
    const float* __restrict__ V = static_cast<const float*>(p.v) + b * p.v_batch + h * kHeadDim;
    float* __restrict__ O = static_cast<float*>(p.o) + b * p.o_batch + h * kHeadDim;
    const uint8_t* __restrict__ KV = mask_reads_valid<MASK>() ? p.key_valid + b * p.kv_batch : nullptr;
    const int rope_tab = p.rope_rows_per_table > 0 ? (p.rope_row0 + b) / p.rope_rows_per_table : 0;
    const float* __restrict__ RC = ROPE ? p.rope_cos + rope_tab * p.rope_table_stride : nullptr;
    const float* __restrict__ RS = ROPE ? p.rope_sin + rope_tab * p.rope_table_stride : nullptr;

    // T5 relative-position bias LUT for this head: lut[j - i + n_q - 1].
    if (BIAS == BIAS_REL) {
        const int n_rel = p.n_q + p.n_k - 1;
        for (int t = tid; t < n_rel; t += 256)
            lut[t] = p.rel_table[min(max(p.rel_bucket[t], 0), p.rel_buckets - 1) * p.H + h];
    }

    // Key range of the workgroup and of this wave (tiles past it are skipped).
    const int wg_qhi = p.q_pos0 + min(p.n_q, q0 + QT) - 1;
    const int kend = key_end_for<MASK>(wg_qhi, p.n_k, p.ctx_keys);
    const int wave_nq = max(0, min(QW, p.n_q - wq0));
    const int wave_kend = wave_nq > 0 ? key_end_for<MASK>(p.q_pos0 + wq0 + wave_nq - 1, p.n_k, p.ctx_keys) : 0;
    const int ntiles = (kend + NK - 1) / NK;
    const int kv_len = valid_len<MASK>(p.n_k, p.ctx_keys);  // key_valid bytes of this row

    // Q^T operand: qreg[qb][s], step s < 8 -> dim 8g+s, s >= 8 -> dim 32+8g+(s-8). Rotated here.
    float qreg[2][16];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int qi = wq0 + 16 * qb + ql;
        f32x4 a0 = {0, 0, 0, 0}, a1 = a0, a2 = a0, a3 = a0;
        if (qi < p.n_q) {
            const float* src = Q + (int64_t)qi * p.q_tok;
            a0 = ld4(src + 8 * g);
            a1 = ld4(src + 8 * g + 4);
            a2 = ld4(src + 32 + 8 * g);
            a3 = ld4(src + 32 + 8 * g + 4);
            if (ROPE) {
                const int64_t row = (int64_t)(p.q_pos0 + qi) * 32;
                const f32x4 c0 = ld4(RC + row + 8 * g), c1 = ld4(RC + row + 8 * g + 4);
                const f32x4 s0 = ld4(RS + row + 8 * g), s1 = ld4(RS + row + 8 * g + 4);
                rope4(a0, a2, c0, s0);
                rope4(a1, a3, c1, s1);
            }
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            qreg[qb][t] = a0[t];
            qreg[qb][4 + t] = a1[t];
            qreg[qb][8 + t] = a2[t];
            qreg[qb][12 + t] = a3[t];
        }
    }

    float m_run[2] = {kNegInf, kNegInf};
    float l_run[2] = {0.f, 0.f};
    f32x4 oacc[4][2];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int qb = 0; qb < 2; qb++) oacc[db][qb] = f32x4{0, 0, 0, 0};

    // Tile loader. K: thread -> (row tid/8 [+32], float4 c4 = tid%8 at dims 4c4 and 32+4c4).
    // V: thread -> (key quad tid/16, dims 4c..4c+3 with c = tid%16), transposed on the way to LDS.
    const int k_row = tid >> 3, k_c4 = tid & 7;
    const int v_kq = tid >> 4, v_c = tid & 15;
    f32x4 kreg[2][2], creg[2], sreg[2], vreg[4];
    uint8_t kvreg = 0;

    auto load_tile = [&](int kbase) {
#pragma unroll
        for (int ps = 0; ps < 2; ps++) {
            const int key = kbase + ps * 32 + k_row;
            if (key < p.n_k) {
                const float* src = K + (int64_t)key * p.k_tok;
                kreg[ps][0] = ld4(src + 4 * k_c4);
                kreg[ps][1] = ld4(src + 32 + 4 * k_c4);
                if (ROPE) {
                    creg[ps] = ld4(RC + (int64_t)key * 32 + 4 * k_c4);
                    sreg[ps] = ld4(RS + (int64_t)key * 32 + 4 * k_c4);
                }
            } else {
                kreg[ps][0] = kreg[ps][1] = f32x4{0, 0, 0, 0};
                if (ROPE) creg[ps] = sreg[ps] = f32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int key = kbase + 4 * v_kq + m;
            vreg[m] = key < p.n_k ? ld4(V + (int64_t)key * p.v_tok + 4 * v_c) : f32x4{0, 0, 0, 0};
        }
        if (mask_reads_valid<MASK>() && tid < NK) kvreg = (kbase + tid < kv_len) ? KV[kbase + tid] : 0;
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int ps = 0; ps < 2; ps++) {
            f32x4 lo = kreg[ps][0], hi = kreg[ps][1];
            if (ROPE) rope4(lo, hi, creg[ps], sreg[ps]);
            float* dst = Ks + (ps * 32 + k_row) * KPAD;
            st4(dst + 4 * k_c4, lo);
            st4(dst + 32 + 4 * k_c4, hi);
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
            st4(Vs + ((v_kq * kHeadDim) + 4 * v_c + j) * 4, f32x4{vreg[0][j], vreg[1][j], vreg[2][j], vreg[3][j]});
        if (mask_reads_valid<MASK>() && tid < NK) kvs[tid] = kvreg;
    };

    if (ntiles > 0) load_tile(0);
    for (int t = 0; t < ntiles; t++) {
        const int kbase = t * NK;
        __syncthreads();
        store_tile();
        __syncthreads();
        if (t + 1 < ntiles) load_tile(kbase + NK);
        if (kbase >= wave_kend) continue;  // nothing left for this wave (uniform)

        // ---- S^T = K . Q^T ----
        f32x4 sacc[4][2];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            const bool kb_on = kbase + kb * 16 < wave_kend;
#pragma unroll
            for (int qb = 0; qb < 2; qb++) sacc[kb][qb] = f32x4{0, 0, 0, 0};
            if (!kb_on) continue;
            const float* kr = Ks + (kb * 16 + ql) * KPAD;
            const f32x4 k0 = ld4(kr + 8 * g), k1 = ld4(kr + 8 * g + 4);
            const f32x4 k2 = ld4(kr + 32 + 8 * g), k3 = ld4(kr + 32 + 8 * g + 4);
            const float kv16[16] = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3],
                                    k2[0], k2[1], k2[2], k2[3], k3[0], k3[1], k3[2], k3[3]};
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                if (16 * qb >= wave_nq) continue;
                f32x4 acc = {0, 0, 0, 0};
#pragma unroll
                for (int s = 0; s < 16; s++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv16[s], qreg[qb][s], acc, 0, 0, 0);
                sacc[kb][qb] = acc;
            }
        }

        // ---- scale, bias, mask, online softmax ----
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            if (16 * qb >= wave_nq) continue;
            const int qi = wq0 + 16 * qb + ql;
            const int qpos = p.q_pos0 + qi;
            float mloc = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const bool kb_on = kbase + kb * 16 < wave_kend;
                uint32_t vw = 0;
                if (mask_reads_valid<MASK>()) vw = *reinterpret_cast<const uint32_t*>(kvs + kb * 16 + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = kbase + kb * 16 + 4 * g + r;
                    float x = kNegInf;
                    if (kb_on) {
#pragma clang fp contract(off)
                        x = sacc[kb][qb][r] * p.scale;
                        if (BIAS == BIAS_REL) x = x + lut[min(max(key - qi + p.n_q - 1, 0), kRelMax - 1)];
                        if (BIAS == BIAS_DENSE && key < p.n_k && qi < p.n_q)
                            x = x + p.bias[h * p.bias_head + (int64_t)qi * p.bias_row + key];
                        x = apply_mask<MASK>(x, key, qpos, p.n_k, ((vw >> (8 * r)) & 0xff) != 0, p.ctx_keys,
                                             p.chain_start);
                    }
                    sacc[kb][qb][r] = x;
                    mloc = fmaxf(mloc, x);
                }
            }
            const float m_new = fmaxf(m_run[qb], rows4_max(mloc));
            const float m_use = m_new == kNegInf ? 0.f : m_new;
            const float alpha = __builtin_amdgcn_exp2f((m_run[qb] - m_use) * kLog2e);
            float lsum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float e = __builtin_amdgcn_exp2f((sacc[kb][qb][r] - m_use) * kLog2e);
                    sacc[kb][qb][r] = e;
                    lsum += e;
                }
            l_run[qb] = l_run[qb] * alpha + lsum;
            m_run[qb] = m_new;
#pragma unroll
            for (int db = 0; db < 4; db++) oacc[db][qb] *= alpha;
        }

        // ---- O^T += V^T . P^T ----
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            if (kbase + kb * 16 >= wave_kend) continue;
#pragma unroll
            for (int db = 0; db < 4; db++) {
                const f32x4 va = ld4(Vs + ((kb * 4 + g) * kHeadDim + db * 16 + ql) * 4);
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    if (16 * qb >= wave_nq) continue;
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        oacc[db][qb] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[r], sacc[kb][qb][r], oacc[db][qb], 0, 0, 0);
                }
            }
        }
    }

    // ---- normalise and store: lane holds query ql, dims 16db + 4g + r ----
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int qi = wq0 + 16 * qb + ql;
        const float l = rows4_sum(l_run[qb]);
        if (qi >= p.n_q) continue;
        const float inv = 1.0f / l;
        float* dst = O + (int64_t)qi * p.o_tok;
#pragma unroll
        for (int db = 0; db < 4; db++) st4(dst + 16 * db + 4 * g, oacc[db][qb] * inv);
    }
}

template <int MASK, int BIAS, bool ROPE>
hipError_t launch_one(const Params& p, hipStream_t stream) {
    const int q_tiles = (p.n_q + QT - 1) / QT;
    const int64_t blocks = (int64_t)p.B * p.H * q_tiles;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fwd_f32<MASK, BIAS, ROPE>), dim3((unsigned)blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
}

template <int MASK, int BIAS>
hipError_t launch_rope(const Params& p, bool rope, hipStream_t s) {
    return rope ? launch_one<MASK, BIAS, true>(p, s) : launch_one<MASK, BIAS, false>(p, s);
}

template <int MASK>
hipError_t launch_bias(const Params& p, int bias, bool rope, hipStream_t s) {
    switch (bias) {
    case BIAS_DENSE: return launch_rope<MASK, BIAS_DENSE>(p, rope, s);
    case BIAS_REL: return launch_rope<MASK, BIAS_REL>(p, rope, s);
    default: return launch_rope<MASK, BIAS_NONE>(p, rope, s);
    }
}

}  // namespace

hipError_t launch_attn_f32(const Params& p, int mask, int bias, bool rope, hipStream_t s) {
    switch (mask) {
    case FULL: return launch_bias<FULL>(p, bias, rope, s);
    case KEYS_ADDITIVE: return launch_bias<KEYS_ADDITIVE>(p, bias, rope, s);
    case CAUSAL: return launch_bias<CAUSAL>(p, bias, rope, s);
    case CAUSAL_KEYS: return launch_bias<CAUSAL_KEYS>(p, bias, rope, s);
    case FULL_KEYS: return launch_bias<FULL_KEYS>(p, bias, rope, s);
    case DECODER: return launch_bias<DECODER>(p, bias, rope, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace tsfm
