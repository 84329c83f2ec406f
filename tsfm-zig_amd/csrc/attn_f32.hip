// f32 attention for short rows (n_k <= 144: Chronos-Bolt's 129-token rows), on the f32 matrix
// cores (v_mfma_f32_16x16x4_f32). Longer rows take the bf16x3 streaming kernel (attn_x3.hip).
//
// The reference computes one (series, head) at a time with a materialised n x n score matrix:
// gemmNT -> bias -> masked softmax -> gemmNN (src/core/attn.zig:72-96). Here the whole batch is one
// launch and no score matrix exists: each (series, head)'s K/V sit in LDS and both products run on
// the matrix cores with an online softmax in registers.
//
// Wave layout (one wave per 16 queries):
//   S^T = K . Q^T   A = K rows (16 keys) from LDS, B = Q^T (16 queries) held in VGPRs.
//                   Accumulator lane l holds query l%16 and keys 4*(l/16)+r, r=0..3.
//   O^T += V^T . P^T  A = V^T (16 dims x 4 keys) from LDS, B = P^T straight from the S^T
//                   accumulator: register r of lane l is key 4*(l/16)+r, exactly the k-slot the
//                   instruction expects, so P never leaves registers.
//   O^T accumulator lane l holds query l%16 and dims 4*(l/16)+r: the same query as the softmax
//   state of that lane, so the online rescale is a plain multiply.
// The contraction order over head dims is permuted (lane group g holds dims 8g..8g+7 and
// 32+8g..32+8g+7) so that every RoPE pair (i, i+32) sits in one lane and K reads are 128-bit.
//
// Accuracy: the f32 matrix instruction rounds after every product, so one 16-step accumulation
// chain over the 64 head dims carries ~2.5x the rounding error of the reference's lane-parallel
// dot product (a few sequential products per SIMD lane, then a tree over lanes). S is therefore
// accumulated in two independent chains of eight instructions, then added: nine rounded steps
// instead of sixteen, within the reference's own cross-host spread, and two dependency chains for
// the matrix pipe. (Four chains of four summed as a tree round six times but cost twelve more VALU
// instructions per 16-key block, and on gfx950 the f32 matrix instructions and the VALU take turns.)
// LDS: K [keys][68] (padded: conflict-free 128-bit reads), V as rows [key][64] (DMA-staged) or
// [key quad][64 dims, XOR-swizzled][4 keys] (register-staged with RoPE), one additive mask term per
// key.
#include <atomic>

#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

constexpr int KPAD = 68;        // K row pitch in LDS (floats)

// Swizzled V slot of a head dim: XOR of bits 3..4 into bits 0..1 spreads both the transposing
// writes (stride 4 dims) and the operand reads (16 consecutive dims) over all LDS banks.
__device__ __forceinline__ int vslot(int dim) { return dim ^ ((dim >> 3) & 3); }

// ---- one wave's 16-query block: state and the per-tile arithmetic ----

// Q^T operand q[s] (step s < 8 -> dim 8g+s, s >= 8 -> dim 32+8g+(s-8) of query ql), the O^T
// accumulator (lane: query ql, dims 16db + 4g + r) and the online-softmax state of the lane's query.
struct QBlock {
    float q[16];
    f32x4 o[4];
    float m;   // running max of the scores
    float ml;  // the same in exp2 units, as used by the weights
    float l;   // running sum of the weights
};

// Load, rotate and scale query qi (zeros past n_q). The score scale goes into q: scores =
// (scale q) . k. For the power-of-two scales every family uses (1, 1/8) this equals the reference's
// alpha * (q . k) bit for bit (scaling by 2^n commutes with every rounding of the dot product).
template <bool ROPE>
__device__ __forceinline__ void load_q(QBlock& w, const float* Q, const float* RC, const float* RS, const Params& p,
                                       int qi, int g) {
    f32x4 a0 = {0, 0, 0, 0}, a1 = a0, a2 = a0, a3 = a0;
    if (qi < p.n_q) {
        const float* src = Q + (int64_t)qi * p.q_tok;
        a0 = ld4(src + 8 * g);
        a1 = ld4(src + 8 * g + 4);
        a2 = ld4(src + 32 + 8 * g);
        a3 = ld4(src + 32 + 8 * g + 4);
        if (ROPE) {
            const int64_t row = (int64_t)(p.q_pos0 + qi) * 32;
            rope4(a0, a2, ld4(RC + row + 8 * g), ld4(RS + row + 8 * g));
            rope4(a1, a3, ld4(RC + row + 8 * g + 4), ld4(RS + row + 8 * g + 4));
        }
        a0 *= p.scale;
        a1 *= p.scale;
        a2 *= p.scale;
        a3 *= p.scale;
    }
#pragma unroll
    for (int t = 0; t < 4; t++) {
        w.q[t] = a0[t];
        w.q[4 + t] = a1[t];
        w.q[8 + t] = a2[t];
        w.q[12 + t] = a3[t];
    }
#pragma unroll
    for (int db = 0; db < 4; db++) w.o[db] = f32x4{0, 0, 0, 0};
    w.m = w.ml = kNegInf;
    w.l = 0.f;
}

// One tile of NKB 16-key blocks for one 16-query block. kt: K rows [key][KPAD] of the tile, vt: its
// V key quads, kat: its key terms, lut: the T5 table (j - i + n_q - 1, readable from -kLutPad to
// n_q + n_k - 1 + kLutPad, so that no index needs a clamp). PLAIN: every key of the tile
// is below n_k and valid, every query past it for the causal masks, so the body has no bounds tests
// and no mask arithmetic; otherwise only the first nkb key blocks are computed and every score goes
// through the mask rule. hook(phase, kb) runs at fixed points (S block kb, after S, PV block kb)
// whether or not the block is computed: the streaming kernel stages the next tile there.
// VROW: vt holds V as rows [key][64] and the O^T accumulator takes the dims in the order
// 16g + 4r + db (register r of w.o[db]): the V operands of one key for the four dim blocks are then
// four consecutive floats of its row (the bits of O are the same; only its register order moves).
template <int MASK, int BIAS, bool PLAIN, int NKB, bool VROW, class Hook>
__device__ __forceinline__ void attend_tile(QBlock& w, const Params& p, const float* kt, const float* vt,
                                            const float* kat, const float* lut, int kbase, int nkb, int qi, int h,
                                            int ql, int g, Hook&& hook) {
    // Lane indices pass through an opaque copy: with both tile variants in one loop the optimiser
    // otherwise hoists every address and key index either variant derives from them out of the
    // loop, and the union of those live ranges spills. The V operand slots are derived here too.
    asm volatile("" : "+v"(g), "+v"(ql), "+v"(qi));
    const int voff_even = vslot(ql) * 4, voff_odd = vslot(16 + ql) * 4;  // V operands, db even / odd

    // ---- S^T = K . Q^T: four accumulation chains per 16-key block, summed as a tree ----
    f32x4 sacc[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; kb++) {
        sacc[kb] = f32x4{0, 0, 0, 0};
        hook(0, kb);
        if (!PLAIN && kb >= nkb) continue;
        const float* kr = kt + (kb * 16 + ql) * KPAD;
        f32x4 c0 = {0, 0, 0, 0}, c1 = c0;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {  // dims 8g.. then 32+8g..: eight K values live at a time
            const f32x4 ka = ld4(kr + 32 * hh + 8 * g), kb4 = ld4(kr + 32 * hh + 8 * g + 4);
            const float* qh = w.q + 8 * hh;
            c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[0], qh[0], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[1], qh[1], c1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[2], qh[2], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[3], qh[3], c1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kb4[0], qh[4], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kb4[1], qh[5], c1, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kb4[2], qh[6], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kb4[3], qh[7], c1, 0, 0, 0);
        }
        sacc[kb] = c0 + c1;
        // Materialise the sum here: left alone, the optimiser sinks it to the softmax and keeps the
        // chain accumulators of the whole tile live.
        asm volatile("" : "+v"(sacc[kb]));
    }
    hook(1, 0);

    // ---- bias, mask, online softmax (the scale is already in q) ----
    {
        // No contraction in this block: ml below must be rounded once and the same value used in the
        // weights and in the rescale (a fused ml_run - m * log2e would mix a rounded and an unrounded
        // maximum: ~1e-6 relative error per rescale, visible at unscaled logits).
#pragma clang fp contract(off)
        const int qpos = p.q_pos0 + qi;
        float mloc = kNegInf;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const bool on = PLAIN || kb < nkb;
            f32x4 ka = {0, 0, 0, 0};
            if (!PLAIN && on) ka = ld4(kat + kb * 16 + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = kbase + kb * 16 + 4 * g + r;
                float x = kNegInf;
                if (on) {
                    x = sacc[kb][r];
                    if (BIAS == BIAS_REL) x = x + lut[key - qi + p.n_q - 1];  // margins: no clamp
                    if (BIAS == BIAS_DENSE && (PLAIN || (key < p.n_k && qi < p.n_q)))
                        x = x + p.bias[h * p.bias_head + (int64_t)qi * p.bias_row + key];
                    if (!PLAIN) x = masked<MASK>(x, ka[r], key, qpos, p.n_k, p.chain_start);
                }
                sacc[kb][r] = x;
                mloc = fmaxf(mloc, x);
            }
        }
        const float m_new = fmaxf(w.m, max4(mloc));
        const float m_use = m_new == kNegInf ? 0.f : m_new;
        // e = exp2(x log2e - m log2e): one FMA per score, with ml = m log2e rounded once and used
        // again by the rescale exp2(ml_old - ml). A row whose max is still an additively masked
        // score (about -FLT_MAX: only invalid keys so far) takes exp2((x - m) log2e) instead, which
        // keeps x - m exact and gives such a row the reference's uniform weights
        // (src/core/nn.zig:470-505 on scores + (-floatMax)).
        const bool big = m_use < -1e30f;
        const float shift = big ? m_use : 0.f;
        const float ml = big ? 0.f : m_use * kLog2e;
        const float alpha = __builtin_amdgcn_exp2f(big ? (w.m - m_use) * kLog2e : w.ml - ml);
        float lsum = 0.f;
        if (__ballot(big) == 0) {  // shift is 0 in every lane: x - shift == x
#pragma unroll
            for (int kb = 0; kb < NKB; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r], kLog2e, -ml));
                    sacc[kb][r] = e;
                    lsum += e;
                }
        } else {
#pragma unroll
            for (int kb = 0; kb < NKB; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r] - shift, kLog2e, -ml));
                    sacc[kb][r] = e;
                    lsum += e;
                }
        }
        w.ml = (big || m_new == kNegInf) ? kNegInf : ml;
        w.l = w.l * alpha + lsum;
        w.m = m_new;
        // Rescale O only when some lane's running max moved (alpha == 1 exactly otherwise).
        if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
            for (int db = 0; db < 4; db++) w.o[db] *= alpha;
        }
    }

    // ---- O^T += V^T . P^T, P straight from the S^T accumulator ----
#pragma unroll
    for (int kb = 0; kb < NKB; kb++) {
        hook(2, kb);
        if (!PLAIN && kb >= nkb) continue;
        if (VROW) {
            // Lane (ql, g), register r: key 16 kb + 4 g + r, dims 4 ql .. 4 ql + 3 (dim block db ->
            // dim 4 ql + db).
            const float* vr = vt + (kb * 16 + 4 * g) * kHeadDim + 4 * ql;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const f32x4 va = ld4(vr + r * kHeadDim);
#pragma unroll
                for (int db = 0; db < 4; db++)
                    w.o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[db], sacc[kb][r], w.o[db], 0, 0, 0);
            }
            continue;
        }
        const float* vq4 = vt + (kb * 4 + g) * (kHeadDim * 4);
#pragma unroll
        for (int dp = 0; dp < 4; dp += 2) {  // two dim blocks at a time: eight V values live
            const f32x4 va0 = ld4(vq4 + dp * 64 + voff_even), va1 = ld4(vq4 + dp * 64 + voff_odd);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                w.o[dp] = __builtin_amdgcn_mfma_f32_16x16x4f32(va0[r], sacc[kb][r], w.o[dp], 0, 0, 0);
                w.o[dp + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(va1[r], sacc[kb][r], w.o[dp + 1], 0, 0, 0);
            }
        }
    }
}

// The last few keys of a row (at most kValuKeys) on the VALU instead of a whole key block of
// matrix instructions: per key, the lane's 16-dim partial dot product (four FMA chains and a tree),
// summed over the query's four lanes, then the same bias, mask and online-softmax update as the
// tile body with one score, and O += e v. Same tile operands in LDS as attend_tile (VROW: V rows
// [key][64] and the O register order of attend_tile's VROW).
constexpr int kValuKeys = 4;
template <int MASK, int BIAS, bool VROW>
__device__ __forceinline__ void attend_keys_valu(QBlock& w, const Params& p, const float* kt, const float* vt,
                                                 const float* kat, const float* lut, int kbase, int nkeys, int qi,
                                                 int h, int g) {
#pragma clang fp contract(off)
    asm volatile("" : "+v"(g), "+v"(qi));  // as in attend_tile: no hoisting out of this variant
    const int qpos = p.q_pos0 + qi;
    for (int j = 0; j < nkeys; j++) {
        const float* kr = kt + j * KPAD;
        const f32x4 k4[4] = {ld4(kr + 8 * g), ld4(kr + 8 * g + 4), ld4(kr + 32 + 8 * g), ld4(kr + 32 + 8 * g + 4)};
        float part[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            part[c] = w.q[4 * c] * k4[c][0];
#pragma unroll
            for (int i = 1; i < 4; i++) part[c] = __builtin_fmaf(w.q[4 * c + i], k4[c][i], part[c]);
        }
        float x = sum4((part[0] + part[1]) + (part[2] + part[3]));
        const int key = kbase + j;
        if (BIAS == BIAS_REL) x = x + lut[key - qi + p.n_q - 1];
        if (BIAS == BIAS_DENSE && key < p.n_k && qi < p.n_q) x = x + p.bias[h * p.bias_head + (int64_t)qi * p.bias_row + key];
        x = masked<MASK>(x, kat[j], key, qpos, p.n_k, p.chain_start);
        const float m_new = fmaxf(w.m, x);
        const float m_use = m_new == kNegInf ? 0.f : m_new;
        const bool big = m_use < -1e30f;
        const float shift = big ? m_use : 0.f;
        const float ml = big ? 0.f : m_use * kLog2e;
        const float alpha = __builtin_amdgcn_exp2f(big ? (w.m - m_use) * kLog2e : w.ml - ml);
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(x - shift, kLog2e, -ml));
        w.ml = (big || m_new == kNegInf) ? kNegInf : ml;
        w.m = m_new;
        w.l = w.l * alpha + (g == 0 ? e : 0.f);  // the query's four lanes share one sum
#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int dim = VROW ? 16 * g + 4 * r + db : 16 * db + 4 * g + r;
                const float vv = VROW ? vt[j * kHeadDim + dim] : vt[(j >> 2) * (kHeadDim * 4) + vslot(dim) * 4 + (j & 3)];
                w.o[db][r] = __builtin_fmaf(e, vv, w.o[db][r] * alpha);
            }
    }
}

// ---- a single query on the VALU ----
//
// A 16-query block that holds one query (n_q = 16k + 1: 577-token Chronos-2 rows, 129-token Bolt
// rows) would spend 15/16 of every matrix instruction on empty query slots. Such a wave takes its
// keys 64 at a time on the VALU instead: lane = key for the score (a 64-term dot product against q,
// read from LDS as a broadcast), one online-softmax step over the chunk with the same update as
// attend_tile, then lane = dim for O += sum_j e_j v_j with the weights broadcast from LDS. The
// running state lives in the QBlock's registers: o[0][0] = O[query, dim lane], m / ml as in
// attend_tile, l = the share of the row sum of the keys this lane has taken.

// DPP lane moves within rows of 16 (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror): combined with max4 / sum4 they reduce over the 64 lanes, every lane getting the
// same value (each step adds two values that are equal up to operand order).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_mov<0xb1>(x));
    x = fmaxf(x, dpp_mov<0x4e>(x));
    x = fmaxf(x, dpp_mov<0x141>(x));
    x = fmaxf(x, dpp_mov<0x140>(x));
    return max4(x);
}
__device__ __forceinline__ float wave_sum(float x) {
    x = x + dpp_mov<0xb1>(x);
    x = x + dpp_mov<0x4e>(x);
    x = x + dpp_mov<0x141>(x);
    x = x + dpp_mov<0x140>(x);
    return sum4(x);
}

// The wave's query (already rotated and scaled in w.q, lanes with ql == 0) to LDS as 64 floats.
__device__ __forceinline__ void thin_store_q(const QBlock& w, float* qs, int ql, int g) {
    if (ql != 0) return;
    st4(qs + 8 * g, f32x4{w.q[0], w.q[1], w.q[2], w.q[3]});
    st4(qs + 8 * g + 4, f32x4{w.q[4], w.q[5], w.q[6], w.q[7]});
    st4(qs + 32 + 8 * g, f32x4{w.q[8], w.q[9], w.q[10], w.q[11]});
    st4(qs + 36 + 8 * g, f32x4{w.q[12], w.q[13], w.q[14], w.q[15]});
}

// Keys kbase .. kbase + nkeys - 1 (1 <= nkeys <= 64) of query qi. kt / vt / kat: the keys' K rows,
// V key quads (VROW: V rows [key][64]) and key terms; qs: the query (thin_store_q); ps: 64 floats of
// LDS for the weights.
template <int MASK, int BIAS, bool VROW = false>
__device__ __forceinline__ void attend_thin(QBlock& w, const Params& p, const float* kt, const float* vt,
                                            const float* kat, const float* lut, const float* qs, float* ps, int kbase,
                                            int nkeys, int qi, int h, int lane) {
#pragma clang fp contract(off)
    asm volatile("" : "+v"(lane));  // as in attend_tile: no hoisting out of this variant
    const int j = min(lane, nkeys - 1);  // lanes past the chunk read a real row; their score is dropped
    const float* kr = kt + j * KPAD;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 16; c++) {
        const f32x4 k4 = ld4(kr + 4 * c), q4 = ld4(qs + 4 * c);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(q4[i], k4[i], acc[i]);
    }
    float x = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    const int key = kbase + j;
    if (BIAS == BIAS_REL) x = x + lut[key - qi + p.n_q - 1];
    if (BIAS == BIAS_DENSE) x = x + p.bias[h * p.bias_head + (int64_t)qi * p.bias_row + key];
    x = masked<MASK>(x, kat[j], key, p.q_pos0 + qi, p.n_k, p.chain_start);
    x = lane < nkeys ? x : kNegInf;

    const float m_new = fmaxf(w.m, wave_max(x));
    const float m_use = m_new == kNegInf ? 0.f : m_new;
    const bool big = m_use < -1e30f;  // as in attend_tile
    const float shift = big ? m_use : 0.f;
    const float ml = big ? 0.f : m_use * kLog2e;
    const float alpha = __builtin_amdgcn_exp2f(big ? (w.m - m_use) * kLog2e : w.ml - ml);
    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(x - shift, kLog2e, -ml));
    w.ml = (big || m_new == kNegInf) ? kNegInf : ml;
    w.m = m_new;
    w.l = w.l * alpha + e;

    ps[lane] = e;  // read back below by the same wave: LDS keeps a wave's accesses in order
    float o = w.o[0][0] * alpha;
    const float* vd = vt + (VROW ? lane : vslot(lane) * 4);
    const int nq4 = (nkeys + 3) >> 2;
    for (int kq = 0; kq < nq4; kq++) {
        const f32x4 p4 = ld4(ps + 4 * kq);
        const f32x4 v4 = VROW ? f32x4{vd[(4 * kq) * kHeadDim], vd[(4 * kq + 1) * kHeadDim], vd[(4 * kq + 2) * kHeadDim],
                                      vd[(4 * kq + 3) * kHeadDim]}
                              : ld4(vd + kq * (kHeadDim * 4));
        o = __builtin_fmaf(p4[0], v4[0], o);
        o = __builtin_fmaf(p4[1], v4[1], o);
        o = __builtin_fmaf(p4[2], v4[2], o);
        o = __builtin_fmaf(p4[3], v4[3], o);
    }
    w.o[0][0] = o;
}

// Normalise and store the single query qi of a thin wave: lane = dim.
__device__ __forceinline__ void store_thin(const QBlock& w, float* O, const Params& p, int qi, int lane) {
    const float l = wave_sum(w.l);
    const float inv = 1.0f / l;
    O[(int64_t)qi * p.o_tok + lane] = w.o[0][0] * inv;
}

// Normalise and store query qi: lane holds dims 16db + 4g + r (VROW: 16g + 4r + db).
template <bool VROW = false>
__device__ __forceinline__ void store_o(const QBlock& w, float* O, const Params& p, int qi, int g) {
    const float l = sum4(w.l);
    if (qi >= p.n_q) return;
    const float inv = 1.0f / l;
    float* dst = O + (int64_t)qi * p.o_tok;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (VROW) st4(dst + 16 * g + 4 * i, f32x4{w.o[0][i], w.o[1][i], w.o[2][i], w.o[3][i]} * inv);
        else st4(dst + 16 * i + 4 * g, w.o[i] * inv);
    }
}

// ---- short rows: every key resident in LDS ------------------------------------------------------
//
// Chronos-Bolt rows are short (at most 128 patches + REG = 129 tokens). Streamed through the
// two-stage pipeline above they pay a staging round and a barrier for each of three tiles, and
// 128-query workgroups leave a one-query tail workgroup (129 = 128 + 1) that stages all of K/V
// again. Here one workgroup of 9 waves (one 16-query block each, 144 queries) loads the whole K, V,
// key terms and T5 table of its (series, head) into LDS once; then every wave runs the per-tile
// arithmetic above over the resident keys with no further barrier. The waves of a workgroup land
// two or three to a SIMD, so two workgroups per CU need room for six waves per SIMD: the kernel is
// built for 80 VGPRs (a few spill to scratch; no global load is in flight there).

constexpr int RNW = 9;                  // waves per workgroup
constexpr int RNT = 64 * RNW;           // threads
constexpr int RQT = 16 * RNW;           // queries per workgroup (144)
constexpr int kResidentKeys = 144;      // longest row the resident kernel takes
constexpr int RNK = 32;                 // keys per tile of the resident loop
constexpr int RKIT = (kResidentKeys * 8 + RNT - 1) / RNT;   // K staging items per thread
constexpr int RVIT = (kResidentKeys * 8 + RNT - 1) / RNT;   // V staging items per thread

// Dynamic LDS layout, in floats: K [nkp][KPAD] | V [nkp/4 quads][64 swizzled][4] | key terms [nkp] |
// T5 table [n_q + n_k - 1 + margins] | a thin wave's q and weights [2][64], with nkp = n_k rounded
// up to 16 keys.
struct ResidentLayout {
    int nkp, v_off, a_off, l_off, t_off, total;
};
__host__ __device__ inline ResidentLayout resident_layout(int n_q, int n_k, bool rel_lut) {
    ResidentLayout L;
    L.nkp = (n_k + 15) & ~15;
    L.v_off = L.nkp * KPAD;
    L.a_off = L.v_off + L.nkp * kHeadDim;
    L.l_off = L.a_off + L.nkp;
    L.t_off = (L.l_off + (rel_lut ? n_q + n_k - 1 + 2 * kLutPad : 0) + 3) & ~3;
    L.total = L.t_off + 2 * kHeadDim;
    return L;
}

template <int MASK, int BIAS, bool ROPE>
__global__ __launch_bounds__(RNT) __attribute__((amdgpu_waves_per_eu(3, 3))) void attn_fwd_f32_resident(Params p,
                                                                                                       int n_items) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const ResidentLayout lay = resident_layout(p.n_q, p.n_k, BIAS == BIAS_REL);

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 15, g = lane >> 4;
    const int q_tiles = (p.n_q + RQT - 1) / RQT;
    const int rope_tabs = p.rope_rows_per_table;

    // Per item (series, head, query tile): the views of its rows. The K / V descriptors end after key
    // n_k - 1, so padding rows up to nkp read as zeros.
    struct Item {
        int b, h, wq0;
        const float* Q;
        const float* K;
        const float* V;
        const float* RC;
        const float* RS;
        __amdgpu_buffer_rsrc_t k_buf, v_buf, c_buf, s_buf, kv_rsrc;
    };
    auto item_of = [&](int it) {
        Item I;
        const int bh = it / q_tiles, qt = it % q_tiles;
        I.b = bh / p.H;
        I.h = bh % p.H;
        I.wq0 = qt * RQT + wave * 16;
        I.Q = static_cast<const float*>(p.q) + I.b * p.q_batch + I.h * kHeadDim;
        const float* K = static_cast<const float*>(p.k) + I.b * p.k_batch + I.h * kHeadDim;
        const float* V = static_cast<const float*>(p.v) + I.b * p.v_batch + I.h * kHeadDim;
        I.K = K;
        I.V = V;
        const int rope_tab = rope_tabs > 0 ? (p.rope_row0 + I.b) / rope_tabs : 0;
        I.RC = ROPE ? p.rope_cos + rope_tab * p.rope_table_stride : nullptr;
        I.RS = ROPE ? p.rope_sin + rope_tab * p.rope_table_stride : nullptr;
        I.k_buf = make_buf(K, (uint32_t)(((int64_t)(p.n_k - 1) * p.k_tok + kHeadDim) * 4));
        I.v_buf = make_buf(V, (uint32_t)(((int64_t)(p.n_k - 1) * p.v_tok + kHeadDim) * 4));
        I.c_buf = make_buf(I.RC, ROPE ? (uint32_t)p.n_k * 128u : 0u);
        I.s_buf = make_buf(I.RS, ROPE ? (uint32_t)p.n_k * 128u : 0u);
        I.kv_rsrc = make_buf(mask_reads_valid<MASK>() ? p.key_valid + I.b * p.kv_batch : p.key_valid,
                             mask_reads_valid<MASK>() ? valid_len<MASK>(p.n_k, p.ctx_keys) : 0);
        return I;
    };

    // ---- staging of one item. Without RoPE (kDma) K and V go from HBM straight into the other LDS
    //      buffer (buffer_load ... lds), so no registers hold them through the compute phase: K as
    //      rows [key][KPAD] (the pad chunk of each row reads zeros out of range), V as rows [key][64]
    //      (the VROW operand order). With RoPE they load into registers, K is rotated at the store
    //      and V is stored key-quad-transposed. q, the T5 table value and the key_valid byte load
    //      into registers either way. ----
    constexpr bool kDma = !ROPE;
    f32x4 klo[RKIT], khi[RKIT], kcs[RKIT], ksn[RKIT];
    f32x4 v01[RVIT], v23[RVIT];
    uint32_t kvb = 1;
    // T5 table entry tid of an item: the bucket of its relative index does not depend on the item,
    // so it is read once here; the item's head picks the table value, loaded with the item's other
    // operands. (Tables longer than the workgroup are filled in stage_store instead.)
    const int n_lut = p.n_q + p.n_k - 1 + 2 * kLutPad;
    const bool lut_in_regs = BIAS == BIAS_REL && n_lut <= RNT;
    int lut_bucket = -1;
    float lut_val = 0.f;
    if (lut_in_regs && tid < n_lut) {
        const int t = min(max(tid - kLutPad, 0), p.n_q + p.n_k - 2);
        lut_bucket = min(max(p.rel_bucket[t], 0), p.rel_buckets - 1);
    }
    f32x4 qa[4];  // the next item's raw q (dims 8g..8g+7, 32+8g..32+8g+7 of query wq0 + ql)
    auto stage_load = [&](const Item& I) {
        // q, the table value and the key_valid byte first, unconditionally (a row past n_q reads
        // the last row and is zeroed at the store): no register they land in waits on the K/V
        // loads issued after them.
        {
            const float* src = I.Q + (int64_t)min(I.wq0 + ql, p.n_q - 1) * p.q_tok;
            qa[0] = ld4(src + 8 * g);
            qa[1] = ld4(src + 8 * g + 4);
            qa[2] = ld4(src + 32 + 8 * g);
            qa[3] = ld4(src + 32 + 8 * g + 4);
        }
        if (lut_bucket >= 0) lut_val = p.rel_table[lut_bucket * p.H + I.h];
        if (mask_reads_valid<MASK>() && tid < lay.nkp) kvb = __builtin_amdgcn_raw_buffer_load_b8(I.kv_rsrc, tid, 0, 0);
        if (kDma) return;
#pragma unroll
        for (int u = 0; u < RKIT; u++) {  // K item = (row, c): dims 4c..4c+3 and 32+4c..32+4c+3
            const int it = tid + u * RNT, row = it >> 3, c = it & 7;
            const uint32_t off = (uint32_t)(row * p.k_tok + 4 * c) * 4u;
            klo[u] = bld4(I.k_buf, off);
            khi[u] = bld4(I.k_buf, off + 128u);
            if (ROPE) {
                const uint32_t coff = (uint32_t)(row * 32 + 4 * c) * 4u;
                kcs[u] = bld4(I.c_buf, coff);
                ksn[u] = bld4(I.s_buf, coff);
            }
        }
#pragma unroll
        for (int u = 0; u < RVIT; u++) {  // V item = (quad of 4 rows, dims 2vc, 2vc+1)
            const int it = tid + u * RNT, quad = it >> 5, vc = it & 31;
            const uint32_t off = (uint32_t)(4 * quad * p.v_tok + 2 * vc) * 4u, step = (uint32_t)p.v_tok * 4u;
            const f32x2 a = bld2(I.v_buf, off), bb = bld2(I.v_buf, off + step);
            const f32x2 c = bld2(I.v_buf, off + 2 * step), d = bld2(I.v_buf, off + 3 * step);
            v01[u] = f32x4{a[0], a[1], bb[0], bb[1]};
            v23[u] = f32x4{c[0], c[1], d[0], d[1]};
        }
    };
    // kDma: the item's K and V into buffer `buf`, 1 KB (64 lanes x 16 bytes) per instruction, the
    // instructions dealt to the waves in turn. K chunk c of the K region is row c / 17, 16-byte piece
    // c % 17 (piece 16: the row's padding); V chunk c is row c / 16, piece c % 16. Rows from n_k up
    // to nkp read as zeros (the descriptors end after key n_k - 1). Issued right after the barrier
    // that released `buf`; read after the wave's `s_waitcnt vmcnt(0)` and the next barrier.
    auto stage_dma = [&](const Item& I, float* buf) {
        const uint32_t lbase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)buf;
        const u32x4 kd = buf_desc(I.K, (uint32_t)(((int64_t)(p.n_k - 1) * p.k_tok + kHeadDim) * 4));
        const u32x4 vd = buf_desc(I.V, (uint32_t)(((int64_t)(p.n_k - 1) * p.v_tok + kHeadDim) * 4));
        const int nk_chunks = lay.nkp * (KPAD / 4), nk_ins = (nk_chunks + 63) / 64;
        const int n_ins = nk_ins + lay.nkp / 4;  // V: nkp rows x 16 pieces = nkp / 4 instructions
        for (int i = wave; i < n_ins; i += RNW) {
            if (i < nk_ins) {
                const int c = 64 * i + lane, row = c / (KPAD / 4), piece = c - row * (KPAD / 4);
                const uint32_t off = piece < kHeadDim / 4 ? (uint32_t)(row * p.k_tok + 4 * piece) * 4u : 0x80000000u;
                if (c < nk_chunks) dma16(kd, lbase + 1024u * i, off, 0u);
            } else {
                const int c = 64 * (i - nk_ins) + lane, row = c >> 4, piece = c & 15;
                dma16(vd, lbase + (uint32_t)lay.v_off * 4u + 1024u * (i - nk_ins),
                      (uint32_t)(row * p.v_tok + 4 * piece) * 4u, 0u);
            }
        }
    };
    // The staged item's remaining parts into buffer `buf` (with registers: K and V too), and the
    // wave's QBlock for it (q rotated and scaled as load_q does).
    auto stage_store = [&](const Item& I, float* buf, QBlock& w) {
        float* const Ks = buf;
        float* const Vs = buf + lay.v_off;
        if (!kDma) {
#pragma unroll
            for (int u = 0; u < RKIT; u++) {
                const int it = tid + u * RNT, row = it >> 3, c = it & 7;
                if (row >= lay.nkp) continue;
                if (ROPE) rope4(klo[u], khi[u], kcs[u], ksn[u]);
                st4(Ks + row * KPAD + 4 * c, klo[u]);
                st4(Ks + row * KPAD + 32 + 4 * c, khi[u]);
            }
#pragma unroll
            for (int u = 0; u < RVIT; u++) {
                const int it = tid + u * RNT, quad = it >> 5, vc = it & 31;
                if (4 * quad >= lay.nkp) continue;
                float* vd = Vs + quad * (kHeadDim * 4);
                st4(vd + vslot(2 * vc) * 4, f32x4{v01[u][0], v01[u][2], v23[u][0], v23[u][2]});
                st4(vd + vslot(2 * vc + 1) * 4, f32x4{v01[u][1], v01[u][3], v23[u][1], v23[u][3]});
            }
        }
        if (tid < lay.nkp) buf[lay.a_off + tid] = key_term<MASK>(tid, p.n_k, kvb != 0, p.ctx_keys);
        if (lut_in_regs) {
            if (lut_bucket >= 0) buf[lay.l_off + tid] = lut_val;
        } else if (BIAS == BIAS_REL) {
            fill_rel_lut(buf + lay.l_off, p, I.h, tid, RNT);
        }
        const int qi = I.wq0 + ql;
        if (qi >= p.n_q) qa[0] = qa[1] = qa[2] = qa[3] = f32x4{0, 0, 0, 0};
        if (ROPE && qi < p.n_q) {
            const int64_t row = (int64_t)(p.q_pos0 + qi) * 32;
            rope4(qa[0], qa[2], ld4(I.RC + row + 8 * g), ld4(I.RS + row + 8 * g));
            rope4(qa[1], qa[3], ld4(I.RC + row + 8 * g + 4), ld4(I.RS + row + 8 * g + 4));
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            w.q[t] = qa[0][t] * p.scale;
            w.q[4 + t] = qa[1][t] * p.scale;
            w.q[8 + t] = qa[2][t] * p.scale;
            w.q[12 + t] = qa[3][t] * p.scale;
        }
#pragma unroll
        for (int db = 0; db < 4; db++) w.o[db] = f32x4{0, 0, 0, 0};
        w.m = w.ml = kNegInf;
        w.l = 0.f;
        if (max(0, min(16, p.n_q - I.wq0)) == 1) thin_store_q(w, buf + lay.t_off, ql, g);
    };

    // ---- one item's attention over the keys resident in `buf` (the store follows separately) ----
    // Offset of key k's V in a buffer's V region: rows (kDma) or key quads.
    auto v_at = [&](const float* Vs, int k) { return Vs + (kDma ? k * kHeadDim : (k >> 2) * (kHeadDim * 4)); };
    auto compute = [&](const Item& I, const float* buf, QBlock& w) {
        const float* const Ks = buf;
        const float* const Vs = buf + lay.v_off;
        const float* const kadd = buf + lay.a_off;
        const float* const lut = buf + lay.l_off + kLutPad;
        float* const thin_qp = const_cast<float*>(buf) + lay.t_off;
        const int wq0 = I.wq0, qi = wq0 + ql, h = I.h;
        const int wave_nq = max(0, min(16, p.n_q - wq0));
        if (wave_nq == 0) return;
        const int wave_kend = key_end_for<MASK>(p.q_pos0 + wq0 + wave_nq - 1, p.n_k, p.ctx_keys);
        if (wave_nq == 1) {  // one query: the VALU path, 64 resident keys at a time
            for (int kb0 = 0; kb0 < wave_kend; kb0 += 64)
                attend_thin<MASK, BIAS, kDma>(w, p, Ks + kb0 * KPAD, v_at(Vs, kb0), kadd + kb0, lut, thin_qp,
                                              thin_qp + kHeadDim, kb0, min(64, wave_kend - kb0), wq0, h, lane);
            return;
        }
        auto no_hook = [](int, int) {};
        // 32-key tiles (two key blocks): half the score registers of a 64-key tile. The last few
        // keys of the row (a tile of at most kValuKeys) go to the VALU after the loop.
        const int klast = wave_kend > 0 ? (wave_kend - 1) / RNK * RNK : 0;
        const int kloop = wave_kend - klast <= kValuKeys ? klast : wave_kend;
        for (int kbase = 0; kbase < kloop; kbase += RNK) {
            const int nkb = min(2, (wave_kend - kbase + 15) >> 4);
            // Query slots past n_q (q = 0, never stored) may run mask-free, except with a dense bias.
            bool plain = kbase + RNK <= wave_kend && (wave_nq == 16 || BIAS != BIAS_DENSE) && MASK != DECODER;
            if (plain && mask_reads_valid<MASK>())
                plain = __ballot(lane < RNK && kadd[kbase + (lane & (RNK - 1))] != 0.f) == 0;
            if (MASK == CAUSAL || MASK == CAUSAL_KEYS) plain = plain && kbase + RNK - 1 <= p.q_pos0 + wq0;
            const float* kt = Ks + kbase * KPAD;
            const float* vt = v_at(Vs, kbase);
            if (plain)
                attend_tile<MASK, BIAS, true, 2, kDma>(w, p, kt, vt, kadd + kbase, lut, kbase, 2, qi, h, ql, g,
                                                       no_hook);
            else
                attend_tile<MASK, BIAS, false, 2, kDma>(w, p, kt, vt, kadd + kbase, lut, kbase, nkb, qi, h, ql, g,
                                                        no_hook);
        }
        if (kloop < wave_kend)
            attend_keys_valu<MASK, BIAS, kDma>(w, p, Ks + kloop * KPAD, v_at(Vs, kloop), kadd + kloop, lut, kloop,
                                               wave_kend - kloop, qi, h, g);
    };
    auto store = [&](const Item& I, const QBlock& w) {
        float* __restrict__ O = static_cast<float*>(p.o) + I.b * p.o_batch + I.h * kHeadDim;
        const int wave_nq = max(0, min(16, p.n_q - I.wq0));
        if (wave_nq == 0) return;
        if (wave_nq == 1) store_thin(w, O, p, I.wq0, lane);
        else store_o<kDma>(w, O, p, I.wq0 + ql, g);
    };

    // ---- persistent loop: item i + gridDim.x stages while item i computes, into the other buffer
    //      (the one item i - gridDim.x used, whose readers all passed the previous barrier); with
    //      registers, its stores follow item i's compute ----
    int it = blockIdx.x;
    if (it >= n_items) return;
    QBlock w;
    Item cur = item_of(it);
    stage_load(cur);
    if (kDma) {
        stage_dma(cur, smem);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    stage_store(cur, smem, w);
    __syncthreads();
    for (int k = 0;; k++) {
        const int nxt = it + gridDim.x;
        const bool more = nxt < n_items;
        float* const nb = smem + ((k + 1) & 1) * lay.total;
        Item next;
        if (more) {
            next = item_of(nxt);
            stage_load(next);
            if (kDma) stage_dma(next, nb);
        }
        compute(cur, smem + (k & 1) * lay.total, w);
        // The next item's LDS copies have landed (waited before this item's O stores are issued, so
        // the wait does not include them).
        if (kDma && more) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        store(cur, w);
        if (!more) break;
        stage_store(next, nb, w);
        // LDS-only barrier: the next item's LDS writes are complete and visible, and every wave has
        // left the buffer the item after it will overwrite. No global access crosses it, so it
        // does not wait for this item's O stores (a __syncthreads() fence would, once per item).
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        cur = next;
        it = nxt;
    }
}

}  // namespace

int device_cus() {
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

namespace {

template <int MASK, int BIAS, bool ROPE>
hipError_t launch_one(const Params& p, hipStream_t stream) {
    const int q_tiles = (p.n_q + RQT - 1) / RQT;
    const int64_t items = (int64_t)p.B * p.H * q_tiles;
    if (items <= 0 || items > 0x7fffffff) return hipErrorInvalidValue;
    const size_t lds = 2 * (size_t)resident_layout(p.n_q, p.n_k, BIAS == BIAS_REL).total * sizeof(float);
    const int cus = device_cus();
    if (cus <= 0) return hipErrorInvalidDevice;
    const int64_t blocks = items < cus ? items : cus;  // one persistent workgroup per CU
    hipLaunchKernelGGL((attn_fwd_f32_resident<MASK, BIAS, ROPE>), dim3((unsigned)blocks), dim3(RNT), lds, stream, p,
                       (int)items);
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
    // Rows longer than the resident kernel takes, and short rows of at least three 32-query blocks
    // in launches of at least two (series, head) pairs per CU: the bf16x3 streaming kernel
    // (attn_x3.hip). Fewer pairs leave its workgroups too few; the resident kernel keeps one per CU.
    if (p.n_k > kResidentKeys || (p.n_q >= 96 && (int64_t)p.B * p.H >= 2 * (int64_t)device_cus()))
        return launch_attn_x3(p, mask, bias, rope, s);
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
