// Fused bf16 / f16 attention with f32 accumulation for gfx950: one workgroup = one (series, head)
// x 128 queries, 4 waves x 32 queries, 64-key tiles.
//
// Same algorithm as attn_f32.hip (the reference's gemmNT -> bias -> masked softmax -> gemmNN,
// src/core/attn.zig:72-96, fused into one pass with an online softmax), on the half-precision
// matrix cores: v_mfma_f32_16x16x32_{f16,bf16}.
//
//   S^T = K . Q^T   A = 16 K rows x 32 dims (lane: key l%16, dims 8*(l/16)..+7) from LDS,
//                   B = Q^T from registers; two instructions cover the 64 head dims. Accumulator
//                   lane l holds query l%16 and keys 4*(l/16)+r.
//   O^T += V^T . P^T  per 32-key chunk: B = P^T packed from the two S^T accumulators of the chunk
//                   (k-slot 8g+j = key 4g+j for j<4, key 16+4g+(j-4) for j>=4), A = V^T from LDS
//                   stored in exactly that key order: [key octet (chunk, g)][dim][8 keys].
// Softmax in f32 registers; P is rounded to the input type for the second product (round to
// nearest even); the row sum is taken on the matrix cores over the same rounded P (ones times P),
// so the weights that are summed are exactly the weights applied to V.
//
// The score scale is folded into the exponent: e = exp2(s * scale*log2(e) - m * scale*log2(e)) is
// one FMA and one v_exp_f32 per score. Tiles below every query's diagonal with all keys valid and
// in range take a body with no mask arithmetic at all: at half precision the matrix cores are 16x
// faster than for f32 and the softmax, not the products, bounds the kernel.
//
// LDS per stage (two stages, one barrier per tile): K [64 keys][72 halves] (padded: conflict-free
// 128-bit operand reads), V [8 octets][64 dims][8 keys] (each staging thread writes whole 16-byte
// slots: conflict-free), the additive mask term of each key, and a per-tile "every key valid" flag.
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int NK = 64;          // keys per tile
constexpr int QW = 32;          // queries per wave
constexpr int NWAVE = 4;
constexpr int NT = 64 * NWAVE;
constexpr int QT = QW * NWAVE;
constexpr int KROW = 36;        // K row pitch in LDS, dwords (64 halves + 8 pad)
constexpr float kStale = 8.f;   // a stale running max may trail the true one by this (exp2 units)

struct StageH {
    uint32_t k[NK * KROW];           // [key][36 dwords]
    uint32_t v[8 * kHeadDim * 4];    // [octet][dim][4 dwords = 8 keys]
    float kadd[NK];
};

template <bool BF16>
__device__ __forceinline__ float lo_f(uint32_t w) {
    if constexpr (BF16) return __uint_as_float(w << 16);
    else return (float)__builtin_bit_cast(f16x2, w)[0];
}
template <bool BF16>
__device__ __forceinline__ float hi_f(uint32_t w) {
    if constexpr (BF16) return __uint_as_float(w & 0xffff0000u);
    else return (float)__builtin_bit_cast(f16x2, w)[1];
}

template <bool BF16>
__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                       0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
}

__device__ __forceinline__ u32x4 ldu4(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// V dim slot within an octet: bit 3 of the dim XORed into bit 0. The staging writes (dims 2dp, then
// 2dp+1, for 8 consecutive dp) and the operand reads (16 consecutive dims, whose slot offset
// vslot_h(db*16 + ql) = db*16 + vslot_h(ql)) then both hit 8 distinct 16-byte bank groups.
__device__ __forceinline__ int vslot_h(int dim) { return dim ^ ((dim >> 3) & 1); }
__device__ __forceinline__ void stu4(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Rotate-half RoPE on 8 dims held as halves: lo = dims i..i+7, hi = dims i+32..i+39, rotated in
// f32 (nn.ropeHalf, src/core/nn.zig:453-460, unfused products) and rounded back.
template <bool BF16>
__device__ __forceinline__ void rope8(u32x4& lo, u32x4& hi, f32x4 c0, f32x4 c1, f32x4 s0, f32x4 s1) {
#pragma clang fp contract(off)
    const float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
    const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    u32x4 nlo, nhi;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const float x1a = lo_f<BF16>(lo[w]), x1b = hi_f<BF16>(lo[w]);
        const float x2a = lo_f<BF16>(hi[w]), x2b = hi_f<BF16>(hi[w]);
        const int i = 2 * w;
        nlo[w] = pack2<BF16>(x1a * cs[i] - x2a * sn[i], x1b * cs[i + 1] - x2b * sn[i + 1]);
        nhi[w] = pack2<BF16>(x2a * cs[i] + x1a * sn[i], x2b * cs[i + 1] + x1b * sn[i + 1]);
    }
    lo = nlo;
    hi = nhi;
}

template <int MASK>
__device__ __forceinline__ float key_term_h(int key, int n_k, bool valid, int ctx_keys) {
    if (key >= n_k) return kNegInf;
    if (MASK == KEYS_ADDITIVE) return valid ? 0.f : -kFltMax;
    if (MASK == CAUSAL_KEYS || MASK == FULL_KEYS) return valid ? 0.f : kNegInf;
    if (MASK == DECODER) return (key < ctx_keys && valid) ? 0.f : kNegInf;
    return 0.f;
}

template <int MASK>
__device__ __forceinline__ float masked_h(float x, float ka, int key, int qpos, int n_k, int chain_start) {
    if (MASK == CAUSAL) return key <= qpos ? x + ka : kNegInf;
    if (MASK == CAUSAL_KEYS) return (key == qpos && key < n_k) ? x : (key <= qpos ? x + ka : kNegInf);
    if (MASK == FULL_KEYS) return (key == qpos && key < n_k) ? x : x + ka;
    if (MASK == DECODER) return (key >= chain_start && key <= qpos && key < n_k) ? x : x + ka;
    return x + ka;
}

// Waves per SIMD the register budget targets: three (168 VGPRs) where the body fits without
// spills, two where RoPE staging or the decoder mask needs more.
template <int MASK, bool ROPE>
constexpr int waves_per_simd() { return (ROPE || MASK == DECODER) ? 2 : 3; }

template <bool BF16, int MASK, bool ROPE>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(waves_per_simd<MASK, ROPE>(),
                                                                   waves_per_simd<MASK, ROPE>()))) void
attn_fwd_half(Params p) {
    __shared__ __attribute__((aligned(16))) StageH stage[2];

    typedef uint16_t E;  // element storage
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

    const E* __restrict__ Q = static_cast<const E*>(p.q) + b * p.q_batch + h * kHeadDim;
    const E* __restrict__ K = static_cast<const E*>(p.k) + b * p.k_batch + h * kHeadDim;
    const E* __restrict__ V = static_cast<const E*>(p.v) + b * p.v_batch + h * kHeadDim;
    E* __restrict__ O = static_cast<E*>(p.o) + b * p.o_batch + h * kHeadDim;
    const uint8_t* __restrict__ KV = mask_reads_valid<MASK>() ? p.key_valid + b * p.kv_batch : nullptr;
    const int rope_tab = p.rope_rows_per_table > 0 ? (p.rope_row0 + b) / p.rope_rows_per_table : 0;
    const float* __restrict__ RC = ROPE ? p.rope_cos + rope_tab * p.rope_table_stride : nullptr;
    const float* __restrict__ RS = ROPE ? p.rope_sin + rope_tab * p.rope_table_stride : nullptr;

    const int wg_qhi = p.q_pos0 + min(p.n_q, q0 + QT) - 1;
    const int kend = key_end_for<MASK>(wg_qhi, p.n_k, p.ctx_keys);
    const int wave_nq = max(0, min(QW, p.n_q - wq0));
    const int wave_qlo = p.q_pos0 + wq0;  // lowest query position of the wave
    const int wave_kend = wave_nq > 0 ? key_end_for<MASK>(p.q_pos0 + wq0 + wave_nq - 1, p.n_k, p.ctx_keys) : 0;
    const int ntiles = (kend + NK - 1) / NK;
    const int kv_len = valid_len<MASK>(p.n_k, p.ctx_keys);
    // exp2 argument factor; KEYS_ADDITIVE keeps the subtract-then-scale form so that the
    // -FLT_MAX terms of an all-invalid row cancel exactly (the reference's uniform row).
    const float c2 = p.scale * kLog2e;

    // Q^T operand: qf[qb][c] = 8 halves, dims 32c + 8g .. 32c + 8g + 7 of query wq0 + 16qb + ql.
    u32x4 qf[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int qi = wq0 + 16 * qb + ql;
        u32x4 lo = {0, 0, 0, 0}, hi = lo;
        if (qi < p.n_q) {
            const E* src = Q + (int64_t)qi * p.q_tok + 8 * g;
            lo = ldu4(src);
            hi = ldu4(src + 32);
            if (ROPE) {
                const int64_t row = (int64_t)(p.q_pos0 + qi) * 32 + 8 * g;
                rope8<BF16>(lo, hi, ld4(RC + row), ld4(RC + row + 4), ld4(RS + row), ld4(RS + row + 4));
            }
        }
        qf[qb][0] = lo;
        qf[qb][1] = hi;
    }

    float mc_run[2] = {kNegInf, kNegInf};  // running max, in exp2 units (max * scale * log2 e)
    // Per query block: the score (same units) past which the running max must move, and the max
    // the exponentials subtract (0 while no key is valid, so that masked scores give e = 0).
    const float slack = MASK == KEYS_ADDITIVE ? kStale / c2 : kStale;
    float thr[2] = {kNegInf, kNegInf}, mc_use[2] = {0.f, 0.f};
    // Row sums on the matrix cores: V^T replaced by ones gives, in every register of the lane,
    // the sum over the chunk's keys of the rounded weights of query ql (the same weights the O
    // product uses). 16 VALU adds per tile and block become one instruction per 32-key chunk.
    f32x4 lacc[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
    const u32x4 ones = BF16 ? u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u}
                            : u32x4{0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u};
    f32x4 oacc[4][2];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int qb = 0; qb < 2; qb++) oacc[db][qb] = f32x4{0, 0, 0, 0};

    // ---- staging: K thread -> key tid/4, dims 8c..8c+7 and 32+8c..32+8c+7 (c = tid%4);
    //      V thread -> dims 2dp, 2dp+1 (dp = tid%32) of the 8 keys of octet tid/32 ----
    // K rows: 16 consecutive lanes take 16 consecutive rows, so each 128-bit LDS write phase of 8
    // lanes covers all banks (row pitch 36 dwords).
    const int krow = (tid & 15) + 16 * (tid >> 6), kc = (tid >> 4) & 3;
    const int dp = tid & 31, oct = tid >> 5;
    const int vkey0 = 32 * (oct >> 2) + 4 * (oct & 3);  // keys vkey0 + {0..3} and vkey0 + 16 + {0..3}
    u32x4 klo, khi;
    f32x4 kc0, kc1, ks0, ks1;  // RoPE cos/sin of the thread's K row, applied at the LDS store
    uint32_t vw[8];
    uint32_t kvb = 1;              // key_valid byte of key kbase + lane of the fetched tile
    float kar = 0.f;
    bool next_all_valid = true;    // uniform: every key term of the fetched tile is 0
    bool next_none_valid = false;  // uniform: no key term of the fetched tile is 0

    // All tile loads go through buffer descriptors that end after key n_k - 1 (key_valid: after
    // the bytes the mask reads): rows of the last tile past the end read as zeros, so no load needs
    // a clamp or a branch, and an offset is one 32-bit VGPR (the host keeps a (series, head) span
    // of K or V below 4 GiB).
    const __amdgpu_buffer_rsrc_t k_buf = make_buf(K, (uint32_t)(((int64_t)(p.n_k - 1) * p.k_tok + kHeadDim) * 2));
    const __amdgpu_buffer_rsrc_t v_buf = make_buf(V, (uint32_t)(((int64_t)(p.n_k - 1) * p.v_tok + kHeadDim) * 2));
    const __amdgpu_buffer_rsrc_t c_buf = make_buf(RC, ROPE ? (uint32_t)p.n_k * 128u : 0u);
    const __amdgpu_buffer_rsrc_t s_buf = make_buf(RS, ROPE ? (uint32_t)p.n_k * 128u : 0u);
    const __amdgpu_buffer_rsrc_t kv_rsrc = make_buf(mask_reads_valid<MASK>() ? KV : p.key_valid,
                                                    mask_reads_valid<MASK>() ? (uint32_t)kv_len : 0u);
    const uint32_t koff = (uint32_t)(krow * p.k_tok + 8 * kc) * 2u;
    const uint32_t voff = (uint32_t)(vkey0 * p.v_tok + 2 * dp) * 2u;
    const uint32_t coff = (uint32_t)(krow * 32 + 8 * kc) * 4u;
    const uint32_t vrow = (uint32_t)p.v_tok * 2u;

    // Loads only: the key terms and the tile flags are derived from kvb in `store`, after the tile
    // being computed, so no wait for this tile's loads sits in front of the products.
    auto fetch = [&](int kbase) {
        const uint32_t kq = koff + (uint32_t)kbase * (uint32_t)p.k_tok * 2u;
        klo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(k_buf, kq, 0, 0));
        khi = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(k_buf, kq + 64u, 0, 0));
        const uint32_t vq = voff + (uint32_t)kbase * vrow;
#pragma unroll
        for (int j = 0; j < 8; j++)
            vw[j] = __builtin_amdgcn_raw_buffer_load_b32(v_buf, vq + (uint32_t)(j < 4 ? j : 12 + j) * vrow, 0, 0);
        if (ROPE) {
            const uint32_t cq = coff + (uint32_t)kbase * 128u;
            kc0 = bld4(c_buf, cq);
            kc1 = bld4(c_buf, cq + 16u);
            ks0 = bld4(s_buf, cq);
            ks1 = bld4(s_buf, cq + 16u);
        }
        if (mask_reads_valid<MASK>()) kvb = __builtin_amdgcn_raw_buffer_load_b8(kv_rsrc, (uint32_t)(kbase + lane), 0, 0);
    };
    auto store = [&](StageH& st, int kbase) {
        {  // every wave evaluates the 64 key terms itself: the tile flags need no LDS round trip
            kar = key_term_h<MASK>(kbase + lane, p.n_k, kvb != 0, p.ctx_keys);
            next_all_valid = __ballot(kar != 0.f) == 0;
            next_none_valid = __ballot(kar == 0.f) == 0;
        }
        if (ROPE) rope8<BF16>(klo, khi, kc0, kc1, ks0, ks1);
        stu4(st.k + krow * KROW + 4 * kc, klo);
        stu4(st.k + krow * KROW + 16 + 4 * kc, khi);
        u32x4 even, odd;  // dims 2dp and 2dp+1, keys in octet order
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t a = vw[2 * w], c = vw[2 * w + 1];
            even[w] = __builtin_amdgcn_perm(c, a, 0x05040100u);  // low halves of a and c
            odd[w] = __builtin_amdgcn_perm(c, a, 0x07060302u);   // high halves
        }
        stu4(st.v + (oct * kHeadDim + vslot_h(2 * dp)) * 4, even);
        stu4(st.v + (oct * kHeadDim + vslot_h(2 * dp + 1)) * 4, odd);
        if (tid < NK) st.kadd[tid] = kar;
    };

    // One 64-key tile on stage st. PLAIN: no mask arithmetic (every key valid and in range, every
    // query of the wave past the tile, all 32 queries in range). Otherwise nkb key blocks and nqb
    // query blocks are computed and each score goes through the mask rule.
    auto tile = [&](const StageH& st, int kbase, int nkb, int nqb, auto plain_tag, int t) {
        constexpr bool PLAIN = decltype(plain_tag)::value;
        const bool more = t + 1 < ntiles;
        if (more) fetch(kbase + NK);

        f32x4 sacc[4][2];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
#pragma unroll
            for (int qb = 0; qb < 2; qb++) sacc[kb][qb] = f32x4{0, 0, 0, 0};
            if (!PLAIN && kb >= nkb) continue;
            const uint32_t* kr = st.k + (kb * 16 + ql) * KROW + 4 * g;
            const u32x4 k0 = ldu4(kr), k1 = ldu4(kr + 16);
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                if (!PLAIN && qb >= nqb) continue;
                sacc[kb][qb] = mfma<BF16>(k1, qf[qb][1], mfma<BF16>(k0, qf[qb][0], sacc[kb][qb]));
            }
        }

        // ---- online softmax in exp2 units ----
        // Per lane and query block, the max of the lane's scores in the units of mc_run (exp2
        // units; raw scores for KEYS_ADDITIVE). The scale is non-negative (checked on the host), so
        // the max of the raw scores times c2 is the max of the scaled ones.
        float mt[2] = {kNegInf, kNegInf};
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            if (!PLAIN && qb >= nqb) continue;
            const int qpos = p.q_pos0 + wq0 + 16 * qb + ql;
            float mloc = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const bool on = PLAIN || kb < nkb;
                f32x4 ka = {0, 0, 0, 0};
                if (!PLAIN) ka = ld4(st.kadd + kb * 16 + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float x = sacc[kb][qb][r];
                    if (!PLAIN) {
                        const int key = kbase + kb * 16 + 4 * g + r;
                        x = on ? masked_h<MASK>(x, ka[r], key, qpos, p.n_k, p.chain_start) : kNegInf;
                    }
                    sacc[kb][qb][r] = x;
                    mloc = fmaxf(mloc, x);
                }
            }
            if (MASK == KEYS_ADDITIVE) mt[qb] = mloc;
            else if (PLAIN) mt[qb] = mloc * c2;  // every score of a mask-free tile is finite
            else mt[qb] = mloc == kNegInf ? kNegInf : mloc * c2;
        }
        // A stale running max is kept until a score exceeds it by more than kStale (exp2 units):
        // weights then stay below 2^kStale, and O and the row sum are rescaled only when some lane
        // of the wave moves past that, rarely after the first tiles of a row. The common case is
        // one compare and a wave-uniform branch per query block; the cross-lane row max is only
        // formed when the running max moves.
        bool upd[2];
#pragma unroll
        for (int qb = 0; qb < 2; qb++) upd[qb] = (PLAIN || qb < nqb) && __ballot(mt[qb] > thr[qb]) != 0;
        if (upd[0] || upd[1]) {
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                if (!upd[qb]) continue;
                const float mk = fmaxf(max4(mt[qb]), mc_run[qb]);  // finite: some score exceeded thr
                const float alpha = MASK == KEYS_ADDITIVE ? __builtin_amdgcn_exp2f((mc_run[qb] - mk) * c2)
                                                          : __builtin_amdgcn_exp2f(mc_run[qb] - mk);
#pragma unroll
                for (int db = 0; db < 4; db++) oacc[db][qb] *= alpha;
                lacc[qb] *= alpha;
                mc_run[qb] = mk;
                thr[qb] = mk + slack;
                mc_use[qb] = mk;
            }
        }
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            if (!PLAIN && qb >= nqb) continue;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float x = sacc[kb][qb][r];
                    sacc[kb][qb][r] = MASK == KEYS_ADDITIVE ? __builtin_amdgcn_exp2f((x - mc_use[qb]) * c2)
                                                            : __builtin_amdgcn_exp2f(__builtin_fmaf(x, c2, -mc_use[qb]));
                }
        }

        // ---- O^T += V^T . P^T, two 32-key chunks ----
#pragma unroll
        for (int ch = 0; ch < 2; ch++) {
            if (!PLAIN && 2 * ch >= nkb) continue;
            u32x4 pf[2];
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                const f32x4 a = sacc[2 * ch][qb], c = sacc[2 * ch + 1][qb];
                pf[qb] = u32x4{pack2<BF16>(a[0], a[1]), pack2<BF16>(a[2], a[3]), pack2<BF16>(c[0], c[1]),
                               pack2<BF16>(c[2], c[3])};
            }
            const uint32_t* vr = st.v + ((ch * 4 + g) * kHeadDim + vslot_h(ql)) * 4;
#pragma unroll
            for (int db = 0; db < 4; db++) {
                const u32x4 vf = ldu4(vr + db * 64);
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    if (!PLAIN && qb >= nqb) continue;
                    oacc[db][qb] = mfma<BF16>(vf, pf[qb], oacc[db][qb]);
                }
            }
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                if (!PLAIN && qb >= nqb) continue;
                lacc[qb] = mfma<BF16>(ones, pf[qb], lacc[qb]);
            }
        }
        // The next tile goes to the other stage last: its loads had the whole tile to land.
        if (more) store(stage[(t + 1) & 1], kbase + NK);
    };

    if (ntiles > 0) {
        fetch(0);
        store(stage[0], 0);
    }
    // Q has landed here on every path (an empty use makes the compiler wait for it now), so no
    // wait for Q is merged into the loop: there, the only loads in flight are the next tile's.
    asm volatile("" : "+v"(qf[0][0]), "+v"(qf[0][1]), "+v"(qf[1][0]), "+v"(qf[1][1]));
    __syncthreads();
    const int nqb = (wave_nq + 15) >> 4;
    for (int t = 0; t < ntiles; t++) {
        const int kbase = t * NK;
        const StageH& st = stage[t & 1];
        const int nkb = min(4, max(0, (wave_kend - kbase + 15) >> 4));
        bool plain = kbase + NK <= wave_kend && wave_nq == QW && MASK != DECODER;
        if (MASK == CAUSAL || MASK == CAUSAL_KEYS) plain = plain && kbase + NK - 1 <= wave_qlo;
        if (mask_reads_valid<MASK>()) plain = plain && next_all_valid;  // fetched with tile t
        // -inf-masked keys contribute nothing: a tile with no valid key and no query's own (always
        // open) diagonal in it is skipped outright (left-padded rows, src/core/attn.zig:46-62).
        const bool empty = (MASK == CAUSAL_KEYS || MASK == FULL_KEYS) && next_none_valid &&
                           (kbase + NK <= wave_qlo || kbase >= wave_qlo + wave_nq);
        if (plain) {
            tile(st, kbase, 4, 2, std::integral_constant<bool, true>{}, t);
        } else if (nkb > 0 && nqb > 0 && !empty) {
            tile(st, kbase, nkb, nqb, std::integral_constant<bool, false>{}, t);
        } else if (t + 1 < ntiles) {
            fetch(kbase + NK);
            store(stage[(t + 1) & 1], kbase + NK);
        }
        __syncthreads();
    }

    // ---- normalise and store: lane holds query ql, dims 16db + 4g + r ----
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int qi = wq0 + 16 * qb + ql;
        const float l = lacc[qb][0];
        if (qi >= p.n_q) continue;
        const float inv = 1.0f / l;
        E* dst = O + (int64_t)qi * p.o_tok + 4 * g;
#pragma unroll
        for (int db = 0; db < 4; db++) {
            const f32x4 o = oacc[db][qb] * inv;
            *reinterpret_cast<u32x2*>(dst + 16 * db) = u32x2{pack2<BF16>(o[0], o[1]), pack2<BF16>(o[2], o[3])};
        }
    }
}

template <bool BF16, int MASK, bool ROPE>
hipError_t launch_one(const Params& p, hipStream_t stream) {
    const int q_tiles = (p.n_q + QT - 1) / QT;
    const int64_t blocks = (int64_t)p.B * p.H * q_tiles;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fwd_half<BF16, MASK, ROPE>), dim3((unsigned)blocks), dim3(NT), 0, stream, p);
    return hipGetLastError();
}

template <bool BF16, int MASK>
hipError_t launch_rope(const Params& p, bool rope, hipStream_t s) {
    return rope ? launch_one<BF16, MASK, true>(p, s) : launch_one<BF16, MASK, false>(p, s);
}

template <bool BF16>
hipError_t launch_mask(const Params& p, int mask, bool rope, hipStream_t s) {
    switch (mask) {
    case FULL: return launch_rope<BF16, FULL>(p, rope, s);
    case KEYS_ADDITIVE: return launch_rope<BF16, KEYS_ADDITIVE>(p, rope, s);
    case CAUSAL: return launch_rope<BF16, CAUSAL>(p, rope, s);
    case CAUSAL_KEYS: return launch_rope<BF16, CAUSAL_KEYS>(p, rope, s);
    case FULL_KEYS: return launch_rope<BF16, FULL_KEYS>(p, rope, s);
    case DECODER: return launch_rope<BF16, DECODER>(p, rope, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_attn_half(const Params& p, bool is_bf16, int mask, int bias, bool rope, hipStream_t s) {
    if (bias != BIAS_NONE) return hipErrorNotSupported;  // the bias-carrying families are f32
    if (!(p.scale >= 0.f)) return hipErrorNotSupported;  // the row max is taken before scaling
    if (attn_half_pipe_supports(p, mask, bias, rope)) return launch_attn_half_pipe(p, is_bf16, mask, s);
    return is_bf16 ? launch_mask<true>(p, mask, rope, s) : launch_mask<false>(p, mask, rope, s);
}

}  // namespace tsfm
