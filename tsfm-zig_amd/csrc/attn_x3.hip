// f32 attention on gfx950's bf16 matrix cores: every f32 operand is split into three bf16 parts
// (a = a0 + a1 + a2, exactly for normal numbers: a0 = bf16(a), a1 = bf16(a - a0), a2 = bf16(a - a0 -
// a1)), and each product a.b is formed from the six partial products whose size is at least 2^-16 of
// |a b| (a2b0, a0b2, a1b1, a1b0, a0b1, a0b0; the three dropped ones are below 2^-24 |a b| together),
// each of them exact in the f32 accumulator. That is the reference's f32 attention
// (src/core/attn.zig:72-96: gemmNT -> bias -> masked softmax -> gemmNN) to within f32 rounding, at
// six bf16 instructions where the f32 matrix instruction (v_mfma_f32_16x16x4_f32) would take the
// time of sixteen, and with the VALU free to run the softmax beside it (the f32 matrix instruction
// and the VALU never overlap on this part; the bf16 one does).
//
// One workgroup = one (series, head) x nw query blocks of 32 (nw waves, 4 to 8), on
// v_mfma_f32_32x32x16_bf16. Per 32-key chunk and wave:
//   S^T = K . Q^T   A = K (lane: key l%32, dims 16s + 8(l/32)..+7), B = Q^T from registers (lane:
//                   query l%32, same dims), four k-steps over the 64 head dims. The five small
//                   products go to one accumulator, the a0b0 products to another; S = big + small.
//                   Accumulator lane l: query l%32, keys 8(r/4) + 4(l/32) + r%4, r < 16.
//   O^T += V^T . P^T  B = P^T split in registers from the lane's own weights (k-slot 8(l/32)+j <->
//                   key 4(l/32) + j for j < 4, 8 + 4(l/32) + j - 4 for j >= 4, in each 16-key half),
//                   A = V^T stored in LDS in that key order; two dim blocks of 32, two k-steps.
//   O^T lane l holds query l%32 (the lane's softmax row) and dims 32db + 8(r/4) + 4(l/32) + r%4.
// Online softmax in f32 registers, exactly the update of the f32 path: a query's 32 scores of a
// chunk sit in lanes l and l ^ 32 (one lane swap for the max; the row sum is combined at the end).
//
// Staging: chunk t + 1 is loaded from HBM into registers while chunk t computes, then split, its K
// RoPE-rotated, and written to the other LDS stage as three bf16 planes: K rows [key][64 dims]
// with 16-byte columns XOR-swizzled by key, V^T rows [dim][32 keys in the operand order] with
// columns swizzled by dim. One barrier per chunk. All HBM reads go through buffer descriptors that
// end after key n_k - 1, so a ragged chunk reads zeros; its keys past n_k carry -inf.
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int XQ = 32;                        // queries per wave
constexpr int XK = 32;                        // keys per chunk
constexpr int XMAXW = 4;                      // waves per workgroup, at most: three per CU
constexpr float kSlack = 5.5f;                // 8 ln 2 - a margin: weights stay below 2^8
constexpr int XMINW = 4;                      // and at least (256 threads: one K and one V item each)
constexpr int XNT = 64 * XMAXW;
constexpr int kPlane = XK * kHeadDim / 2;     // dwords per bf16 plane of a chunk's K or V (4 KB)

struct XStage {
    uint32_t k[3][kPlane];  // [plane][key][8 x 16-byte columns; column c holds dims 8c..8c+7 at c ^ (key & 7)]
    uint32_t v[3][kPlane];  // [plane][dim][4 x 16-byte columns; column 2j + h at (2j + h) ^ ((dim >> 2) & 3)]
    float kadd[XK];         // additive mask term of each key of the chunk
};

__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}
__device__ __forceinline__ u32x4 lds16(const uint32_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Two values as three bf16 parts, each word holding the pair (first value in the low half):
// h = bf16(a), m = bf16(a - h), l = bf16(a - h - m), round to nearest even. a - h and the next
// remainder are exact in f32; they are formed as a + (-1) h by v_dot2_f32_bf16 (one instruction
// instead of a widening shift and a subtraction), with the (-1, 0) and (0, -1) operands in
// registers: the compiler would encode (-1, 0) as the inline constant -1.0, which the instruction
// does not read as that pair.
struct NegOne {
    bf16x2 lo, hi;  // (-1, 0) and (0, -1)
};
__device__ __forceinline__ NegOne neg_one() {
    uint32_t lo = 0x0000bf80u, hi = 0xbf800000u;
    asm volatile("" : "+v"(lo), "+v"(hi));
    return NegOne{__builtin_bit_cast(bf16x2, lo), __builtin_bit_cast(bf16x2, hi)};
}
struct Split {
    uint32_t h, m, l;
};
__device__ __forceinline__ Split split2(float a, float b, NegOne n) {
    Split r;
    r.h = pack2<true>(a, b);
    const float ra = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, r.h), n.lo, a, false);
    const float rb = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, r.h), n.hi, b, false);
    r.m = pack2<true>(ra, rb);
    r.l = pack2<true>(__builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, r.m), n.lo, ra, false),
                      __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, r.m), n.hi, rb, false));
    return r;
}
// Four values as three bf16 planes.
__device__ __forceinline__ void split4(f32x4 v, u32x2& hi, u32x2& mid, u32x2& lo, NegOne n) {
    const Split a = split2(v[0], v[1], n), b = split2(v[2], v[3], n);
    hi = u32x2{a.h, b.h};
    mid = u32x2{a.m, b.m};
    lo = u32x2{a.l, b.l};
}
// 1 for a row of 32k + 1 queries that one workgroup takes (1 <= k <= 8): its last query runs
// outside the 32-query blocks, at the end of the workgroup, instead of as a 32-query block of its own
// (longer rows keep that block: there the pass would lengthen one workgroup in three).
__host__ __device__ inline int thin_query(int n_q) { return (n_q > XQ && n_q <= XMAXW * XQ + 1 && n_q % XQ == 1) ? 1 : 0; }

__device__ __forceinline__ float pair_max(float x) {  // lanes l and l ^ 32
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

template <int MASK, int BIAS, bool ROPE>
__global__ __launch_bounds__(XNT) __attribute__((amdgpu_waves_per_eu(3, 3))) void attn_fwd_x3(Params p) {
    __shared__ __attribute__((aligned(16))) XStage stage[2];
    extern __shared__ float lut_raw[];  // the T5 table (n_q + n_k - 1 + margins), sized at launch
    float* const lut = lut_raw + (BIAS == BIAS_REL ? kLutPad : 0);

    const int nt = blockDim.x, nw = nt >> 6;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int qt_n = nw * XQ;
    // A row of 32k + 1 queries: the 32-query blocks take the first 32k, and the last query runs on
    // the VALU at the start of the workgroup of the last blocks (see below).
    const int thin = thin_query(p.n_q);
    const int n_main = p.n_q - thin;
    const int q_tiles = (n_main + qt_n - 1) / qt_n;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = logical / q_tiles;
    int qt = logical % q_tiles;
    if (MASK == CAUSAL || MASK == CAUSAL_KEYS) qt = q_tiles - 1 - qt;  // longest rows first
    const int b = bh / p.H, h = bh % p.H;
    const int q0 = qt * qt_n;
    const int wq0 = q0 + wave * XQ;
    const int qi = wq0 + ql;

    const float* __restrict__ Q = static_cast<const float*>(p.q) + b * p.q_batch + h * kHeadDim;
    const float* __restrict__ K = static_cast<const float*>(p.k) + b * p.k_batch + h * kHeadDim;
    const float* __restrict__ V = static_cast<const float*>(p.v) + b * p.v_batch + h * kHeadDim;
    float* __restrict__ O = static_cast<float*>(p.o) + b * p.o_batch + h * kHeadDim;
    const int rope_tab = p.rope_rows_per_table > 0 ? (p.rope_row0 + b) / p.rope_rows_per_table : 0;
    const float* __restrict__ RC = ROPE ? p.rope_cos + rope_tab * p.rope_table_stride : nullptr;
    const float* __restrict__ RS = ROPE ? p.rope_sin + rope_tab * p.rope_table_stride : nullptr;

    // Key range of the workgroup (chunks past it are not staged) and of this wave.
    const int wg_qhi = p.q_pos0 + min(n_main, q0 + qt_n) - 1;
    const int kend = key_end_for<MASK>(wg_qhi, p.n_k, p.ctx_keys);
    const int wave_nq = max(0, min(XQ, n_main - wq0));
    const int wave_kend = wave_nq > 0 ? key_end_for<MASK>(p.q_pos0 + wq0 + wave_nq - 1, p.n_k, p.ctx_keys) : 0;
    // Rows of 32k + 1 keys under the masks whose key range is the whole row: the last key on the VALU
    // after the chunks (one dot product per query instead of a 32-key chunk of matrix work).
    const bool tail_key = (MASK == FULL || MASK == KEYS_ADDITIVE || MASK == FULL_KEYS) && p.n_k % XK == 1 && p.n_k > 1;
    const int nchunks = tail_key ? p.n_k / XK : (kend + XK - 1) / XK;

    const __amdgpu_buffer_rsrc_t kv_rsrc = make_buf(mask_reads_valid<MASK>() ? p.key_valid + b * p.kv_batch : p.key_valid,
                                                    mask_reads_valid<MASK>() ? valid_len<MASK>(p.n_k, p.ctx_keys) : 0);
    const __amdgpu_buffer_rsrc_t k_buf = make_buf(K, (uint32_t)(((int64_t)(p.n_k - 1) * p.k_tok + kHeadDim) * 4));
    const __amdgpu_buffer_rsrc_t v_buf = make_buf(V, (uint32_t)(((int64_t)(p.n_k - 1) * p.v_tok + kHeadDim) * 4));
    const __amdgpu_buffer_rsrc_t c_buf = make_buf(RC, ROPE ? (uint32_t)p.n_k * 128u : 0u);
    const __amdgpu_buffer_rsrc_t s_buf = make_buf(RS, ROPE ? (uint32_t)p.n_k * 128u : 0u);

    // ---- staging. K item (threads tid < 256): key row tid >> 3, dims 4c..4c+3 and 32+4c..32+4c+3 with
    //      c = tid & 7 (a RoPE pair). V item (threads tid >= nt - 256, x = tid - (nt - 256)): key quad
    //      x >> 5, dims 2(x & 31) and 2(x & 31) + 1. Both roles are uniform per wave; with 256
    //      threads every thread has one of each. ----
    const NegOne neg = neg_one();
    const bool k_role = tid < 256;
    const int vx_item = tid - (nt - 256);
    const bool v_role = vx_item >= 0;
    const int kr_item = tid >> 3, kc_item = tid & 7;
    // V quads with bits 0 and 1 of vx_item >> 5 swapped: the two half-waves of a wave then write
    // different 8-byte halves of their 16-byte columns, which halves the LDS bank conflicts of the
    // V stores (a store's lanes spread over twice the banks).
    const int vq_item = ((vx_item >> 5) & 4) | (((vx_item >> 5) & 1) << 1) | ((vx_item >> 6) & 1), vd_item = vx_item & 31;
    f32x4 k_lo, k_hi, k_cs, k_sn;  // K item: dims lo / hi and, with RoPE, its rotation
    f32x4 v_01, v_23;              // V item: keys 0, 1 / keys 2, 3 of the quad, (dim, dim + 1) pairs
    uint32_t kvb = 1;              // key_valid byte of key tid of the chunk being staged (threads < 32)
    auto load_chunk = [&](int kb) {
        if (k_role) {
            const uint32_t off = (uint32_t)((kb + kr_item) * p.k_tok + 4 * kc_item) * 4u;
            k_lo = bld4(k_buf, off);
            k_hi = bld4(k_buf, off + 128u);
            if (ROPE) {
                const uint32_t coff = (uint32_t)((kb + kr_item) * 32 + 4 * kc_item) * 4u;
                k_cs = bld4(c_buf, coff);
                k_sn = bld4(s_buf, coff);
            }
        }
        if (v_role) {
            const uint32_t off = (uint32_t)((kb + 4 * vq_item) * p.v_tok + 2 * vd_item) * 4u;
            const uint32_t step = (uint32_t)p.v_tok * 4u;
            const f32x2 v0 = bld2(v_buf, off), v1 = bld2(v_buf, off + step);
            const f32x2 v2 = bld2(v_buf, off + 2 * step), v3 = bld2(v_buf, off + 3 * step);
            v_01 = f32x4{v0[0], v0[1], v1[0], v1[1]};
            v_23 = f32x4{v2[0], v2[1], v3[0], v3[1]};
        }
        if (mask_reads_valid<MASK>() && tid < XK) kvb = __builtin_amdgcn_raw_buffer_load_b8(kv_rsrc, kb + tid, 0, 0);
    };
    auto store_chunk = [&](XStage& st, int kb) {
        u32x2 p0, p1, p2;
        if (k_role) {
            if (ROPE) rope4(k_lo, k_hi, k_cs, k_sn);
            const int row = kr_item * 32 + 2 * (kc_item & 1), sw = kr_item & 7;
            const int lo = row + (((kc_item >> 1) ^ sw) << 2), hi = row + (((4 + (kc_item >> 1)) ^ sw) << 2);
            split4(k_lo, p0, p1, p2, neg);
            *reinterpret_cast<u32x2*>(&st.k[0][lo]) = p0;
            *reinterpret_cast<u32x2*>(&st.k[1][lo]) = p1;
            *reinterpret_cast<u32x2*>(&st.k[2][lo]) = p2;
            split4(k_hi, p0, p1, p2, neg);
            *reinterpret_cast<u32x2*>(&st.k[0][hi]) = p0;
            *reinterpret_cast<u32x2*>(&st.k[1][hi]) = p1;
            *reinterpret_cast<u32x2*>(&st.k[2][hi]) = p2;
        }
        if (v_role) {
            const int col = 2 * (vq_item >> 2) + (vq_item & 1), wo = 2 * ((vq_item >> 1) & 1);
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = 2 * vd_item + e;
                const int off = d * 16 + ((col ^ ((d >> 2) & 3)) << 2) + wo;
                split4(f32x4{v_01[e], v_01[2 + e], v_23[e], v_23[2 + e]}, p0, p1, p2, neg);
                *reinterpret_cast<u32x2*>(&st.v[0][off]) = p0;
                *reinterpret_cast<u32x2*>(&st.v[1][off]) = p1;
                *reinterpret_cast<u32x2*>(&st.v[2][off]) = p2;
            }
        }
        if (tid < XK) st.kadd[tid] = key_term<MASK>(kb + tid, p.n_k, kvb != 0, p.ctx_keys);
    };

    // ---- the wave's queries: rotated, scaled (the scale is a power of two in every family, so
    //      (scale q) . k is the reference's alpha (q . k) bit for bit) and split ----
    if (BIAS == BIAS_REL) fill_rel_lut(lut_raw, p, h, tid, nt);
    if (thin && qt == q_tiles - 1) {
        // ---- the single query past the blocks (n_q = 32k + 1), in the workgroup of the last blocks,
        //      before the blocks' own work: each wave takes a slice of the keys from K / V in global
        //      memory on the VALU (bringing them into L2 for the staging that follows), lane = key for
        //      the scores and lane = dim for O; the slices' maxima, sums and partial rows are merged
        //      through LDS. Weights exp2((x - m) log2e), exact for rows that only have additively
        //      masked scores so far (the reference's uniform weights). ----
        // In the second stage's K parts, first written at the end of chunk 0 (after the barrier that
        // follows the staging of chunk 0, which wave 0 reaches once its merge is done): the query, a
        // wave's weights of a 64-key batch and then its partial row, a wave's max and sum.
        float* const tq = reinterpret_cast<float*>(stage[1].k[0]);
        float (*const tw)[kHeadDim] = reinterpret_cast<float (*)[kHeadDim]>(tq + kHeadDim);
        float (*const tml)[2] = reinterpret_cast<float (*)[2]>(tq + kHeadDim + XMAXW * kHeadDim);
        static_assert((1 + XMAXW) * kHeadDim + 2 * XMAXW <= kPlane, "the single-query pass fits one K part");
        const int qn = p.n_q - 1, qposn = p.q_pos0 + qn;
        const int kend_n = key_end_for<MASK>(qposn, p.n_k, p.ctx_keys);
        if (wave == 0 && lane < 32) {
    #pragma clang fp contract(off)
            float x1 = Q[(int64_t)qn * p.q_tok + lane], x2 = Q[(int64_t)qn * p.q_tok + lane + 32];
            if (ROPE) {  // nn.ropeHalf, src/core/nn.zig:453-460
                const float c = RC[(int64_t)qposn * 32 + lane], sn = RS[(int64_t)qposn * 32 + lane];
                const float y1 = x1 * c - x2 * sn, y2 = x2 * c + x1 * sn;
                x1 = y1;
                x2 = y2;
            }
            tq[lane] = x1 * p.scale;
            tq[lane + 32] = x2 * p.scale;
        }
        __syncthreads();
        const int per = (kend_n + nw - 1) / nw, k0 = wave * per, k1 = min(kend_n, k0 + per);
        float mw = kNegInf, lw = 0.f, ow = 0.f;
        for (int kb = k0; kb < k1; kb += 64) {
    #pragma clang fp contract(off)
            const int key = kb + lane;
            float x = kNegInf;
            if (key < k1) {
                const float* kr = K + (int64_t)key * p.k_tok;
                float acc = 0.f;
    #pragma unroll
                for (int c = 0; c < 8; c++) {
                    f32x4 lo = ld4(kr + 4 * c), hi = ld4(kr + 32 + 4 * c);
                    if (ROPE) rope4(lo, hi, ld4(RC + (int64_t)key * 32 + 4 * c), ld4(RS + (int64_t)key * 32 + 4 * c));
                    const f32x4 qa = ld4(tq + 4 * c), qb = ld4(tq + 32 + 4 * c);
    #pragma unroll
                    for (int i = 0; i < 4; i++) acc = __builtin_fmaf(qb[i], hi[i], __builtin_fmaf(qa[i], lo[i], acc));
                }
                x = acc;
                if (BIAS == BIAS_REL) x = x + lut[key];  // relative index key - qn + n_q - 1 = key
                if (BIAS == BIAS_DENSE) x = x + p.bias[h * p.bias_head + (int64_t)qn * p.bias_row + key];
                const uint32_t kvb = mask_reads_valid<MASK>() ? __builtin_amdgcn_raw_buffer_load_b8(kv_rsrc, key, 0, 0) : 1u;
                x = masked<MASK>(x, key_term<MASK>(key, p.n_k, kvb != 0, p.ctx_keys), key, qposn, p.n_k, p.chain_start);
            }
            float cm = x;
    #pragma unroll
            for (int o2 = 32; o2 > 0; o2 >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o2));
            const float mn = fmaxf(mw, cm);
            if (mn == kNegInf) continue;  // wave-uniform: nothing to weigh yet
            const float alpha = mw == kNegInf ? 0.f : __builtin_amdgcn_exp2f((mw - mn) * kLog2e);
            const float e = key < k1 ? __builtin_amdgcn_exp2f((x - mn) * kLog2e) : 0.f;
            lw = lw * alpha + e;  // the lane's share of the slice's sum
            ow = ow * alpha;
            tw[wave][lane] = e;  // read back by the same wave: LDS keeps a wave's accesses in order
            // O += sum_j e_j v_j, sixteen rows' loads in flight at a time (rows past the slice carry
            // weight 0 and read the slice's last row).
            const int nk = min(64, k1 - kb);
            const float* vr = V + (int64_t)kb * p.v_tok + lane;
            for (int j0 = 0; j0 < nk; j0 += 16) {
                float vv[16];
    #pragma unroll
                for (int i = 0; i < 16; i++) vv[i] = vr[(int64_t)min(j0 + i, nk - 1) * p.v_tok];
    #pragma unroll
                for (int i = 0; i < 16; i++) ow = __builtin_fmaf(j0 + i < nk ? tw[wave][j0 + i] : 0.f, vv[i], ow);
            }
            mw = mn;
        }
    #pragma unroll
        for (int o2 = 32; o2 > 0; o2 >>= 1) lw += __shfl_xor(lw, o2);
        if (lane == 0) {
            tml[wave][0] = mw;
            tml[wave][1] = lw;
        }
        tw[wave][lane] = ow;
        __syncthreads();
        if (wave == 0) {
        float M = kNegInf;
        for (int w = 0; w < nw; w++) M = fmaxf(M, tml[w][0]);
        float L = 0.f, acc = 0.f;
        for (int w = 0; w < nw; w++) {
            if (tml[w][0] == kNegInf) continue;
            const float sw = __builtin_amdgcn_exp2f((tml[w][0] - M) * kLog2e);
            L = L + tml[w][1] * sw;
            acc = acc + tw[w][lane] * sw;
        }
        O[(int64_t)qn * p.o_tok + lane] = acc / L;
        }

    }
    load_chunk(0);
    u32x4 qf[3][4];  // [plane][k-step]: dims 16s + 8 hh .. +7 of query qi
    {
        f32x4 qa[4][2];
        const float* src = Q + (int64_t)min(qi, n_main - 1) * p.q_tok;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            qa[s][0] = ld4(src + 16 * s + 8 * hh);
            qa[s][1] = ld4(src + 16 * s + 8 * hh + 4);
        }
        if (ROPE) {
            const int64_t row = (int64_t)(p.q_pos0 + min(qi, n_main - 1)) * 32;
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int i = 0; i < 2; i++)
                    rope4(qa[s][i], qa[s + 2][i], ld4(RC + row + 16 * s + 8 * hh + 4 * i),
                          ld4(RS + row + 16 * s + 8 * hh + 4 * i));
        }
        const float sc = qi < n_main ? p.scale : 0.f;  // query slots past the blocks: q = 0, never stored
#pragma unroll
        for (int s = 0; s < 4; s++) {
            u32x2 a0, a1, a2, b0, b1, b2;
            split4(qa[s][0] * sc, a0, a1, a2, neg);
            split4(qa[s][1] * sc, b0, b1, b2, neg);
            qf[0][s] = u32x4{a0[0], a0[1], b0[0], b0[1]};
            qf[1][s] = u32x4{a1[0], a1[1], b1[0], b1[1]};
            qf[2][s] = u32x4{a2[0], a2[1], b2[0], b2[1]};
        }
    }
    // The tail key's K row (rotated, as the staged rows are) and V row, and its key term.
    __shared__ __attribute__((aligned(16))) float ktail[kHeadDim], vtail[kHeadDim];
    __shared__ float tail_add;
    if (tail_key && tid < kHeadDim) {
        const int kt = p.n_k - 1;
        if (tid < 32) {
#pragma clang fp contract(off)
            float x1 = K[(int64_t)kt * p.k_tok + tid], x2 = K[(int64_t)kt * p.k_tok + tid + 32];
            if (ROPE) {  // nn.ropeHalf, src/core/nn.zig:453-460
                const float c = RC[(int64_t)kt * 32 + tid], sn = RS[(int64_t)kt * 32 + tid];
                const float y1 = x1 * c - x2 * sn, y2 = x2 * c + x1 * sn;
                x1 = y1;
                x2 = y2;
            }
            ktail[tid] = x1;
            ktail[tid + 32] = x2;
        }
        vtail[tid] = V[(int64_t)kt * p.v_tok + tid];
        if (tid == 0) {
            const bool valid = mask_reads_valid<MASK>() ? p.key_valid[b * p.kv_batch + kt] != 0 : true;
            tail_add = key_term<MASK>(kt, p.n_k, valid, p.ctx_keys);
        }
    }
    store_chunk(stage[0], 0);
    __syncthreads();

    f32x16 o[2] = {f32x16{}, f32x16{}};
    float m = kNegInf, ml = kNegInf, l = 0.f;
    const int qpos = p.q_pos0 + qi;
    const int qc = min(qi, p.n_q - 1);  // the T5 row of a query slot past n_q (its scores are dropped)
    const int kx = ql & 7, vx = (ql >> 2) & 3;

    // Online update for a new score max mc of the lane's query: the weights' reference max m trails
    // the running max by at most kSlack, so a max that stays within it leaves m, ml, l and O as they
    // are (weights up to 2^8; the normalised result is the same) and O is rescaled in few chunks.
    // Returns the shift and the exp2-unit max the weights are formed against; shifted: some lane
    // of the wave needs the shift.
    auto update = [&](float mc, float& shift, float& mlw, bool& shifted) {
#pragma clang fp contract(off)
        shift = 0.f;
        mlw = ml;
        shifted = false;
        if (__ballot(!(m > -1e30f && mc <= m + kSlack)) != 0) {
            const float m_new = fmaxf(m, mc);
            const float m_use = m_new == kNegInf ? 0.f : m_new;
            // As the f32 path: e = exp2(x log2e - m log2e) with ml = m log2e rounded once; a row whose
            // max is still an additively masked score (about -FLT_MAX) takes exp2((x - m) log2e),
            // which gives it the reference's uniform weights (src/core/nn.zig:470-505 on scores +
            // (-floatMax)).
            const bool big = m_use < -1e30f;
            shift = big ? m_use : 0.f;
            mlw = big ? 0.f : m_use * kLog2e;
            const float alpha = __builtin_amdgcn_exp2f(big ? (m - m_use) * kLog2e : ml - mlw);
            ml = (big || m_new == kNegInf) ? kNegInf : mlw;
            l = l * alpha;
            m = m_new;
            shifted = __ballot(big) != 0;
            if (__ballot(alpha != 1.f) != 0) {
                o[0] *= alpha;
                o[1] *= alpha;
            }
        }
    };

    for (int t = 0; t < nchunks; t++) {
        const int kbase = t * XK;
        const XStage& st = stage[t & 1];
        const bool more = t + 1 < nchunks;
        if (more) load_chunk(kbase + XK);
        if (kbase < wave_kend) {
            // ---- S^T = K . Q^T: the twenty small products first, then the four a0 b0 ones, into one
            //      accumulator (the small terms round at their own size, the large ones four times) ----
            f32x16 sacc = {};
            u32x4 k0[4];
            const uint32_t* kr0 = st.k[0] + ql * 32;
            const uint32_t* kr1 = st.k[1] + ql * 32;
            const uint32_t* kr2 = st.k[2] + ql * 32;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int col = ((2 * s + hh) ^ kx) << 2;
                k0[s] = lds16(kr0 + col);
                const u32x4 k1 = lds16(kr1 + col), k2 = lds16(kr2 + col);
                sacc = mfma32(k2, qf[0][s], sacc);
                sacc = mfma32(k0[s], qf[2][s], sacc);
                sacc = mfma32(k1, qf[1][s], sacc);
                sacc = mfma32(k1, qf[0][s], sacc);
                sacc = mfma32(k0[s], qf[1][s], sacc);
            }
#pragma unroll
            for (int s = 0; s < 4; s++) sacc = mfma32(k0[s], qf[0][s], sacc);
            // Mask-free chunk: every key below wave_kend (<= n_k) and valid and, for the causal masks,
            // at or before every query of the wave. Query slots past n_q may run mask-free too,
            // except with a dense bias (no bias row to read).
            bool plain = kbase + XK <= wave_kend && (wave_nq == XQ || BIAS != BIAS_DENSE) && MASK != DECODER;
            if (plain && mask_reads_valid<MASK>()) plain = __ballot(st.kadd[lane & 31] != 0.f) == 0;
            if (MASK == CAUSAL || MASK == CAUSAL_KEYS) plain = plain && kbase + XK - 1 <= p.q_pos0 + wq0;

            // ---- bias, mask, online softmax (the scale is already in q) ----
            u32x4 pf[3][2];  // P^T planes, [plane][k-step]
            {
#pragma clang fp contract(off)
                float x[16];
                float mloc = kNegInf;
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const f32x4 ka = plain ? f32x4{0, 0, 0, 0} : ld4(st.kadd + 8 * g4 + 4 * hh);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = 4 * g4 + i, key = kbase + 8 * g4 + 4 * hh + i;
                        float v = sacc[r];
                        if (BIAS == BIAS_REL) v = v + lut[key - qc + p.n_q - 1];  // margins: no clamp
                        if (BIAS == BIAS_DENSE && (plain || (key < p.n_k && qi < p.n_q)))
                            v = v + p.bias[h * p.bias_head + (int64_t)qi * p.bias_row + key];
                        if (!plain) v = masked<MASK>(v, ka[i], key, qpos, p.n_k, p.chain_start);
                        x[r] = v;
                        mloc = fmaxf(mloc, v);
                    }
                }
                float shift, mlw;
                bool shifted;
                update(pair_max(mloc), shift, mlw, shifted);
                float lsum = 0.f;
                if (!shifted) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(x[r], kLog2e, -mlw));
                        x[r] = e;
                        lsum += e;
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(x[r] - shift, kLog2e, -mlw));
                        x[r] = e;
                        lsum += e;
                    }
                }
                l = l + lsum;
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        const Split t = split2(x[8 * j + 2 * w], x[8 * j + 2 * w + 1], neg);
                        pf[0][j][w] = t.h;
                        pf[1][j][w] = t.m;
                        pf[2][j][w] = t.l;
                    }
            }

            // ---- O^T += V^T . P^T ----
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int col = ((2 * j + hh) ^ vx) << 2;
#pragma unroll
                for (int db = 0; db < 2; db++) {
                    const int off = (32 * db + ql) * 16 + col;
                    const u32x4 v0 = lds16(st.v[0] + off), v1 = lds16(st.v[1] + off), v2 = lds16(st.v[2] + off);
                    o[db] = mfma32(v2, pf[0][j], o[db]);
                    o[db] = mfma32(v0, pf[2][j], o[db]);
                    o[db] = mfma32(v1, pf[1][j], o[db]);
                    o[db] = mfma32(v1, pf[0][j], o[db]);
                    o[db] = mfma32(v0, pf[1][j], o[db]);
                    o[db] = mfma32(v0, pf[0][j], o[db]);
                }
            }
        }
        // Chunk t + 1 goes to the other stage, last read in chunk t - 1 (every wave has passed the
        // barrier after it).
        if (more) store_chunk(stage[(t + 1) & 1], kbase + XK);
        __syncthreads();
    }

    // ---- normalise and store: lane (ql, hh) holds dims 32db + 8g + 4hh .. +3 of query qi ----
    if (tail_key && wave_nq > 0) {
#pragma clang fp contract(off)
        // The lane's 32 dims of its query, exactly, from the three parts (hi + mid, then lo), and
        // their share of the dot product with the tail key; the pair of lanes adds the halves.
        auto part = [](uint32_t w, int half) { return __uint_as_float(half ? (w & 0xffff0000u) : (w << 16)); };
        float acc = 0.f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const f32x4 k0 = ld4(ktail + 16 * s + 8 * hh), k1 = ld4(ktail + 16 * s + 8 * hh + 4);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int w = j >> 1, hf = j & 1;
                const float qv = (part(qf[0][s][w], hf) + part(qf[1][s][w], hf)) + part(qf[2][s][w], hf);
                acc = __builtin_fmaf(qv, j < 4 ? k0[j] : k1[j - 4], acc);
            }
        }
        const int key = p.n_k - 1;
        float x = pair_sum(acc);
        if (BIAS == BIAS_REL) x = x + lut[key - qc + p.n_q - 1];
        if (BIAS == BIAS_DENSE && qi < p.n_q) x = x + p.bias[h * p.bias_head + (int64_t)qi * p.bias_row + key];
        x = masked<MASK>(x, tail_add, key, qpos, p.n_k, p.chain_start);
        float shift, mlw;
        bool shifted;
        update(x, shift, mlw, shifted);
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(x - shift, kLog2e, -mlw));
        l = l + (hh == 0 ? e : 0.f);  // the pair shares one key
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const f32x4 v4 = ld4(vtail + 32 * db + 8 * g4 + 4 * hh);
#pragma unroll
                for (int i = 0; i < 4; i++) o[db][4 * g4 + i] = __builtin_fmaf(e, v4[i], o[db][4 * g4 + i]);
            }
    }
    const float lt = pair_sum(l);
    if (wave_nq > 0) {
        // Through the wave's own 8 KB of the stages (idle since the loop's last barrier), so that a
        // store instruction writes four whole 256-byte rows: row r's 16-byte column c sits at
        // c ^ (r & 15), which keeps both the writes and the reads free of bank conflicts.
        float* const ob = reinterpret_cast<float*>(&stage[0]) + wave * (XQ * kHeadDim);
        const float inv = 1.0f / lt;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int c = 8 * db + 2 * g4 + hh;
                *reinterpret_cast<f32x4*>(ob + ql * kHeadDim + 4 * (c ^ (ql & 15))) =
                    f32x4{o[db][4 * g4], o[db][4 * g4 + 1], o[db][4 * g4 + 2], o[db][4 * g4 + 3]} * inv;
            }
        const int c = lane & 15;
#pragma unroll
        for (int k = 0; k < XQ / 4; k++) {
            const int r = (lane >> 4) + 4 * k;
            if (r < wave_nq)
                st4(O + (int64_t)(wq0 + r) * p.o_tok + 4 * c,
                    *reinterpret_cast<const f32x4*>(ob + r * kHeadDim + 4 * (c ^ (r & 15))));
        }
    }

}

template <int MASK, int BIAS, bool ROPE>
hipError_t launch_one(const Params& p, hipStream_t stream) {
    const int n_main = p.n_q - thin_query(p.n_q);
    const int qb = (n_main + XQ - 1) / XQ;
    const int q_tiles = (qb + XMAXW - 1) / XMAXW;
    const int nw = max(XMINW, (qb + q_tiles - 1) / q_tiles);
    const int64_t blocks = (int64_t)p.B * p.H * ((n_main + nw * XQ - 1) / (nw * XQ));
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    const size_t lut_bytes = BIAS == BIAS_REL ? (size_t)(p.n_q + p.n_k - 1 + 2 * kLutPad) * sizeof(float) : 0;
    hipLaunchKernelGGL((attn_fwd_x3<MASK, BIAS, ROPE>), dim3((unsigned)blocks), dim3(64 * nw), lut_bytes, stream, p);
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

hipError_t launch_attn_x3(const Params& p, int mask, int bias, bool rope, hipStream_t s) {
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
