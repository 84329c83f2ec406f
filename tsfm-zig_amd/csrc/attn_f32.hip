// Fused f32 attention for gfx950: one workgroup = one (series, head) x 128 queries.
//
// The reference computes one (series, head) at a time with a materialised n x n score matrix:
// gemmNT -> bias -> masked softmax -> gemmNN (src/core/attn.zig:72-96). Here the whole batch is one
// launch and no score matrix exists: K/V tiles of 64 keys are staged in LDS and both products run
// on the f32 matrix cores (v_mfma_f32_16x16x4_f32) with an online softmax in registers.
//
// Wave layout (8 waves x 16 queries; four waves per SIMD hide each other's latencies):
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
// accumulated in four independent chains of four instructions, summed as a tree, which brings the
// scores to the reference's accuracy and gives the matrix pipe four independent dependency chains.
//
// Pipeline: two LDS stages. While the waves compute on stage t&1, tile t+1 is fetched from HBM and
// written to the other stage in two 32-key halves (one over the S product, one over softmax and
// the PV product), 13 registers per thread; one barrier per tile. The whole wave state (q, O,
// scores, operands, staging) fits 128 registers, which gives four waves per SIMD.
// LDS per stage: K [64 keys][68] (padded: conflict-free 128-bit reads), V [16 key quads][64 dims,
// XOR-swizzled][4 keys] (conflict-free transposing writes and operand reads), and one additive mask
// term per key. Two stages + the T5 table fit two workgroups per CU.
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

constexpr int NK = 64;          // keys per LDS tile
constexpr int QW = 16;          // queries per wave (one 16-query block)
constexpr int NWAVE = 8;
constexpr int NT = 64 * NWAVE;  // threads per workgroup
constexpr int QT = QW * NWAVE;  // queries per workgroup
constexpr int KPAD = 68;        // K row pitch in LDS (floats)

struct Stage {
    float k[NK * KPAD];      // [key][KPAD], RoPE applied
    float v[NK * kHeadDim];  // [key quad][swizzled dim][4 keys]
    float kadd[NK];          // additive mask term of each key (0, -FLT_MAX or -inf)
};

// Swizzled V slot of a head dim: XOR of bits 3..4 into bits 0..1 spreads both the transposing
// writes (stride 4 dims) and the operand reads (16 consecutive dims) over all LDS banks.
__device__ __forceinline__ int vslot(int dim) { return dim ^ ((dim >> 3) & 3); }

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

template <int MASK, int BIAS, bool ROPE>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4, 4))) void attn_fwd_f32(Params p) {
    __shared__ __attribute__((aligned(16))) Stage stage[2];
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
    const int rope_tab = p.rope_rows_per_table > 0 ? (p.rope_row0 + b) / p.rope_rows_per_table : 0;
    const float* __restrict__ RC = ROPE ? p.rope_cos + rope_tab * p.rope_table_stride : nullptr;
    const float* __restrict__ RS = ROPE ? p.rope_sin + rope_tab * p.rope_table_stride : nullptr;

    // Key range of the workgroup and of this wave (tiles past it are skipped).
    const int wg_qhi = p.q_pos0 + min(p.n_q, q0 + QT) - 1;
    const int kend = key_end_for<MASK>(wg_qhi, p.n_k, p.ctx_keys);
    const int wave_nq = max(0, min(QW, p.n_q - wq0));
    const int wave_kend = wave_nq > 0 ? key_end_for<MASK>(p.q_pos0 + wq0 + wave_nq - 1, p.n_k, p.ctx_keys) : 0;
    const int ntiles = (kend + NK - 1) / NK;

    // key_valid of this row through a buffer descriptor sized to the bytes the mask reads: a read
    // past them returns 0 (= invalid), so the load needs neither a bounds test nor a branch.
    const __amdgpu_buffer_rsrc_t kv_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(mask_reads_valid<MASK>() ? p.key_valid + b * p.kv_batch : p.key_valid), (short)0,
        mask_reads_valid<MASK>() ? valid_len<MASK>(p.n_k, p.ctx_keys) : 0, kBufferConfig);

    // Q^T operand: qreg[s], step s < 8 -> dim 8g+s, s >= 8 -> dim 32+8g+(s-8) of query wq0 + ql,
    // rotated and scaled in the prologue.
    float qreg[16];
    float m_run = kNegInf;   // running max of the scores
    float ml_run = kNegInf;  // the same in exp2 units, as used by the weights
    float l_run = 0.f;
    f32x4 oacc[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};

    // ---- tile staging: HBM -> registers -> LDS, one 16-key quarter at a time (6 registers) ----
    // K: thread -> key row tid/32 of the quarter, dims c and c+32 with c = tid%32 (a RoPE pair).
    // V: wave w -> half w%2 of key quad w/2 of the quarter, lane -> dim: two keys of one dim, half
    //    of a 16-byte slot of the transposed layout. Key valid bytes: lane = key of the tile, in every
    //    wave, with the tile's first quarter.
    // All through buffer descriptors that end after key n_k - 1: rows past it (tile padding) read
    // as zeros, so a partial tile needs no clamping and no branch.
    const int krow = tid >> 5, kc = tid & 31;
    struct Quarter {  // one thread's share of a 16-key quarter tile, in flight from HBM to LDS
        float klo, khi, kcs, ksn;
        f32x2 v;  // V rows 4*(wave/2) + 2*(wave%2) + 0..1 of the quarter, dim `lane`
    };
    const __amdgpu_buffer_rsrc_t k_buf = make_buf(K, (uint32_t)(((int64_t)(p.n_k - 1) * p.k_tok + kHeadDim) * 4));
    const __amdgpu_buffer_rsrc_t v_buf = make_buf(V, (uint32_t)(((int64_t)(p.n_k - 1) * p.v_tok + kHeadDim) * 4));
    const __amdgpu_buffer_rsrc_t c_buf = make_buf(RC, ROPE ? (uint32_t)p.n_k * 128u : 0u);
    const __amdgpu_buffer_rsrc_t s_buf = make_buf(RS, ROPE ? (uint32_t)p.n_k * 128u : 0u);
    const uint32_t koff = (uint32_t)(krow * p.k_tok + kc) * 4u;
    const uint32_t voff = (uint32_t)((4 * (wave >> 1) + 2 * (wave & 1)) * p.v_tok + lane) * 4u;
    const uint32_t coff = (uint32_t)(krow * 32 + kc) * 4u;

    auto fetch = [&](int qbase, Quarter& hs) {  // keys [qbase, qbase + 16)
        const uint32_t kq = koff + (uint32_t)(qbase * p.k_tok) * 4u;
        hs.klo = bld1(k_buf, kq);
        hs.khi = bld1(k_buf, kq + 128u);
        const uint32_t vq = voff + (uint32_t)(qbase * p.v_tok) * 4u;
        hs.v = f32x2{bld1(v_buf, vq), bld1(v_buf, vq + (uint32_t)p.v_tok * 4u)};
        if (ROPE) {
            hs.kcs = bld1(c_buf, coff + (uint32_t)qbase * 128u);
            hs.ksn = bld1(s_buf, coff + (uint32_t)qbase * 128u);
        }
    };
    auto store = [&](Stage& st, int quarter, Quarter& hs) {
        if (ROPE) {
#pragma clang fp contract(off)
            const float x1 = hs.klo, x2 = hs.khi;  // nn.ropeHalf, src/core/nn.zig:453-460
            hs.klo = x1 * hs.kcs - x2 * hs.ksn;
            hs.khi = x2 * hs.kcs + x1 * hs.ksn;
        }
        float* kd = st.k + (quarter * 16 + krow) * KPAD + kc;
        kd[0] = hs.klo;
        kd[32] = hs.khi;
        st2(st.v + (quarter * 4 + (wave >> 1)) * (kHeadDim * 4) + vslot(lane) * 4 + 2 * (wave & 1), hs.v);
    };
    // key_valid byte of key tbase + lane (returned as loaded; 1 for masks that do not read it).
    auto fetch_valid = [&](int tbase) -> uint32_t {
        return mask_reads_valid<MASK>() ? __builtin_amdgcn_raw_buffer_load_b8(kv_rsrc, tbase + lane, 0, 0) : 1u;
    };
    // Additive mask term of key tbase + lane, and the tile's mask-free test (every term 0).
    auto kterm = [&](int tbase, uint32_t kvb) { return key_term<MASK>(tbase + lane, p.n_k, kvb != 0, p.ctx_keys); };
    auto all_valid = [&](int tbase, uint32_t kvb) { return __ballot(kterm(tbase, kvb) != 0.f) == 0; };
    uint32_t kvb_next;  // key_valid bytes of the tile being staged

    // V operand offsets of this lane (floats, within a key quad): dim db*16 + ql, swizzled.
    const int voff_even = vslot(ql) * 4, voff_odd = vslot(16 + ql) * 4;  // db even / odd

    // One 64-key tile on stage `st`. PLAIN: every key of the tile is below n_k and valid, every
    // query of the wave below n_q and, for the causal masks, past the tile, so the body has no
    // bounds tests and no mask arithmetic; otherwise only the first nkb key blocks are computed
    // (uniform) and every score goes through the mask rule.
    auto tile = [&](const Stage& st, int kbase, int nkb, auto plain_tag, int t) {
        constexpr bool PLAIN = decltype(plain_tag)::value;
        const bool more = t + 1 < ntiles;
        Stage& nxt = stage[(t + 1) & 1];
        const int nbase = kbase + NK;
        Quarter sq;  // the next tile's quarters pass through here, one per quarter of this tile's work
        if (more) {
            fetch(nbase, sq);
            kvb_next = fetch_valid(nbase);
        }

        // ---- S^T = K . Q^T, four accumulation chains per 16-key block ----
        f32x4 sacc[4];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            sacc[kb] = f32x4{0, 0, 0, 0};
            if (more && (kb == 1 || kb == 3)) {  // next tile: quarter kb/2 to LDS, fetch the next one
                store(nxt, kb >> 1, sq);
                fetch(nbase + 16 * (kb / 2 + 1), sq);
            }
            if (!PLAIN && kb >= nkb) continue;
            const float* kr = st.k + (kb * 16 + ql) * KPAD;
            f32x4 c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {  // dims 8g.. then 32+8g..: eight K values live at a time
                const f32x4 ka = ld4(kr + 32 * hh + 8 * g), kb4 = ld4(kr + 32 * hh + 8 * g + 4);
                const float* qh = qreg + 8 * hh;
                c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[0], qh[0], c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[1], qh[1], c1, 0, 0, 0);
                c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[2], qh[2], c2, 0, 0, 0);
                c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[3], qh[3], c3, 0, 0, 0);
                c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kb4[0], qh[4], c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kb4[1], qh[5], c1, 0, 0, 0);
                c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(kb4[2], qh[6], c2, 0, 0, 0);
                c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(kb4[3], qh[7], c3, 0, 0, 0);
            }
            sacc[kb] = (c0 + c1) + (c2 + c3);
            // Materialise the sum here: left alone, the optimiser sinks it to the softmax and keeps
            // the chain accumulators of the whole tile live.
            asm volatile("" : "+v"(sacc[kb]));
        }
        if (more) nxt.kadd[lane] = kterm(nbase, kvb_next);  // every wave writes the same 64 terms

        // ---- bias, mask, online softmax (the scale is already in q) ----
        {
            // No contraction in this block: ml below must be rounded once and the same value used in
            // the weights and in the rescale (a fused ml_run - m * log2e would mix a rounded and an
            // unrounded maximum: ~1e-6 relative error per rescale, visible at unscaled logits).
#pragma clang fp contract(off)
            const int qi = wq0 + ql;
            const int qpos = p.q_pos0 + qi;
            float mloc = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const bool on = PLAIN || kb < nkb;
                f32x4 ka = {0, 0, 0, 0};
                if (!PLAIN && on) ka = ld4(st.kadd + kb * 16 + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = kbase + kb * 16 + 4 * g + r;
                    float x = kNegInf;
                    if (on) {
                        x = sacc[kb][r];
                        if (BIAS == BIAS_REL) x = x + lut[min(max(key - qi + p.n_q - 1, 0), kRelMax - 1)];
                        if (BIAS == BIAS_DENSE && (PLAIN || (key < p.n_k && qi < p.n_q)))
                            x = x + p.bias[h * p.bias_head + (int64_t)qi * p.bias_row + key];
                        if (!PLAIN) x = masked<MASK>(x, ka[r], key, qpos, p.n_k, p.chain_start);
                    }
                    sacc[kb][r] = x;
                    mloc = fmaxf(mloc, x);
                }
            }
            const float m_new = fmaxf(m_run, max4(mloc));
            const float m_use = m_new == kNegInf ? 0.f : m_new;
            // e = exp2(x log2e - m log2e): one FMA per score. The running max is kept in exp2 units
            // (ml_run), so the rescale uses the same rounded values as the weights. A row whose max
            // is still an additively masked score (about -FLT_MAX: only invalid keys so far) takes
            // exp2((x - m) log2e) instead, which keeps x - m exact and gives such a row the
            // reference's uniform weights (src/core/nn.zig:470-505 on scores + (-floatMax)).
            const bool big = m_use < -1e30f;
            const float shift = big ? m_use : 0.f;
            const float ml = big ? 0.f : m_use * kLog2e;
            const float alpha = __builtin_amdgcn_exp2f(big ? (m_run - m_use) * kLog2e : ml_run - ml);
            float lsum = 0.f;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r] - shift, kLog2e, -ml));
                    sacc[kb][r] = e;
                    lsum += e;
                }
            ml_run = (big || m_new == kNegInf) ? kNegInf : ml;
            l_run = l_run * alpha + lsum;
            m_run = m_new;
            // Rescale O only when some lane's running max moved (alpha == 1 exactly otherwise).
            if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
                for (int db = 0; db < 4; db++) oacc[db] *= alpha;
            }
        }

        // ---- O^T += V^T . P^T ----
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            if (more && kb == 2) {
                store(nxt, 2, sq);
                fetch(nbase + 48, sq);
            }
            if (!PLAIN && kb >= nkb) continue;
            const float* vq4 = st.v + (kb * 4 + g) * (kHeadDim * 4);
#pragma unroll
            for (int dp = 0; dp < 4; dp += 2) {  // two dim blocks at a time: eight V values live
                const f32x4 va0 = ld4(vq4 + dp * 64 + voff_even), va1 = ld4(vq4 + dp * 64 + voff_odd);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    oacc[dp] = __builtin_amdgcn_mfma_f32_16x16x4f32(va0[r], sacc[kb][r], oacc[dp], 0, 0, 0);
                    oacc[dp + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(va1[r], sacc[kb][r], oacc[dp + 1], 0, 0, 0);
                }
            }
        }
        if (more) store(nxt, 3, sq);
    };

    // Prologue: tile 0's two halves, q and the T5 table are all requested before anything waits,
    // so a short row pays about one memory latency here, not several.
    kvb_next = fetch_valid(0);
    Quarter s0, s1, s2, s3;
    fetch(0, s0);
    fetch(16, s1);
    fetch(32, s2);
    fetch(48, s3);
    {
        const int qi = wq0 + ql;
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
            // The score scale goes into q: scores = (scale q) . k. For the power-of-two scales every
            // family uses (1, 1/8) this equals the reference's alpha * (q . k) bit for bit (scaling
            // by 2^n commutes with every rounding of the dot product).
            a0 *= p.scale;
            a1 *= p.scale;
            a2 *= p.scale;
            a3 *= p.scale;
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            qreg[t] = a0[t];
            qreg[4 + t] = a1[t];
            qreg[8 + t] = a2[t];
            qreg[12 + t] = a3[t];
        }
    }
    if (BIAS == BIAS_REL) {  // lut[j - i + n_q - 1] for this head, two entries per thread per round
        const int n_rel = p.n_q + p.n_k - 1;
        for (int t0 = 0; t0 < n_rel; t0 += 2 * NT) {
            int bk[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int t = t0 + u * NT + tid;
                bk[u] = t < n_rel ? min(max(p.rel_bucket[t], 0), p.rel_buckets - 1) : 0;
            }
            float val[2];
#pragma unroll
            for (int u = 0; u < 2; u++) val[u] = p.rel_table[bk[u] * p.H + h];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int t = t0 + u * NT + tid;
                if (t < n_rel) lut[t] = val[u];
            }
        }
    }
    store(stage[0], 0, s0);
    store(stage[0], 1, s1);
    store(stage[0], 2, s2);
    store(stage[0], 3, s3);
    stage[0].kadd[lane] = kterm(0, kvb_next);
    bool next_all_valid = all_valid(0, kvb_next);  // of the tile about to be computed
    __syncthreads();
    for (int t = 0; t < ntiles; t++) {
        const int kbase = t * NK;
        const Stage& st = stage[t & 1];
        const int nkb = min(4, max(0, (wave_kend - kbase + 15) >> 4));
        // Mask-free tile: all 64 keys below wave_kend (<= n_k) and valid, all 16 queries below n_q
        // and, for the causal masks, at or past the tile's last key.
        bool plain = kbase + NK <= wave_kend && wave_nq == QW && MASK != DECODER && next_all_valid;
        if (MASK == CAUSAL || MASK == CAUSAL_KEYS) plain = plain && kbase + NK - 1 <= p.q_pos0 + wq0;
        if (plain) {
            tile(st, kbase, 4, std::integral_constant<bool, true>{}, t);
        } else if (nkb > 0) {
            tile(st, kbase, nkb, std::integral_constant<bool, false>{}, t);
        } else if (t + 1 < ntiles) {
            Stage& nxt = stage[(t + 1) & 1];
            kvb_next = fetch_valid(kbase + NK);
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                Quarter sq;
                fetch(kbase + NK + 16 * qq, sq);
                store(nxt, qq, sq);
            }
            nxt.kadd[lane] = kterm(kbase + NK, kvb_next);
        }
        // The next tile's flag, from its key_valid bytes fetched at the start of this one.
        if (t + 1 < ntiles) next_all_valid = all_valid(kbase + NK, kvb_next);
        __syncthreads();
    }

    // ---- normalise and store: lane holds query ql, dims 16db + 4g + r ----
    const int qi = wq0 + ql;
    const float l = sum4(l_run);
    if (qi < p.n_q) {
        const float inv = 1.0f / l;
        float* dst = O + (int64_t)qi * p.o_tok;
#pragma unroll
        for (int db = 0; db < 4; db++) st4(dst + 16 * db + 4 * g, oacc[db] * inv);
    }
}

// ---- short rows: every key resident in LDS ------------------------------------------------------
//
// Chronos-Bolt rows are short (at most 128 patches + REG = 129 tokens). Streamed through the
// two-stage pipeline above they pay a staging round and a barrier for each of three tiles, and
// 128-query workgroups leave a one-query tail workgroup (129 = 128 + 1) that stages all of K/V
// again. Here one workgroup of 3 waves x 3 query blocks (144 queries) loads the whole K, V, key
// terms and T5 table of its (series, head) into LDS once, then runs the same per-tile arithmetic
// (four-chain scores, online softmax, P kept in registers) without any further barrier.

constexpr int RQB = 3;                  // query blocks of 16 per wave
constexpr int RNW = 3;                  // waves per workgroup
constexpr int RNT = 64 * RNW;           // threads
constexpr int RQT = 16 * RQB * RNW;     // queries per workgroup (144)
constexpr int kResidentKeys = 144;      // longest row the resident kernel takes
constexpr int RKIT = (kResidentKeys * 8 + RNT - 1) / RNT;  // K staging items per thread
constexpr int RVIT = (kResidentKeys * 8 + RNT - 1) / RNT;  // V staging items per thread

// Dynamic LDS layout, in floats: K [nkp][KPAD] | V [nkp/4 quads][64 swizzled][4] | key terms [nkp] |
// T5 table [n_q + n_k - 1], with nkp = n_k rounded up to 16 keys.
struct ResidentLayout {
    int nkp, v_off, a_off, l_off, total;
};
__host__ __device__ inline ResidentLayout resident_layout(int n_q, int n_k, bool rel_lut) {
    ResidentLayout L;
    L.nkp = (n_k + 15) & ~15;
    L.v_off = L.nkp * KPAD;
    L.a_off = L.v_off + L.nkp * kHeadDim;
    L.l_off = L.a_off + L.nkp;
    L.total = L.l_off + (rel_lut ? n_q + n_k - 1 : 0);
    return L;
}

template <int MASK, int BIAS, bool ROPE>
__global__ __launch_bounds__(RNT) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_f32_resident(Params p) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const ResidentLayout lay = resident_layout(p.n_q, p.n_k, BIAS == BIAS_REL);
    float* const Ks = smem;
    float* const Vs = smem + lay.v_off;
    float* const kadd = smem + lay.a_off;
    float* const lut = smem + lay.l_off;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ql = lane & 15, g = lane >> 4;
    const int q_tiles = (p.n_q + RQT - 1) / RQT;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = logical / q_tiles, qt = logical % q_tiles;
    const int b = bh / p.H, h = bh % p.H;
    const int wq0 = qt * RQT + wave * 16 * RQB;  // first query of this wave

    const float* __restrict__ Q = static_cast<const float*>(p.q) + b * p.q_batch + h * kHeadDim;
    const float* __restrict__ K = static_cast<const float*>(p.k) + b * p.k_batch + h * kHeadDim;
    const float* __restrict__ V = static_cast<const float*>(p.v) + b * p.v_batch + h * kHeadDim;
    float* __restrict__ O = static_cast<float*>(p.o) + b * p.o_batch + h * kHeadDim;
    const uint8_t* __restrict__ KV = mask_reads_valid<MASK>() ? p.key_valid + b * p.kv_batch : nullptr;
    const int rope_tab = p.rope_rows_per_table > 0 ? (p.rope_row0 + b) / p.rope_rows_per_table : 0;
    const float* __restrict__ RC = ROPE ? p.rope_cos + rope_tab * p.rope_table_stride : nullptr;
    const float* __restrict__ RS = ROPE ? p.rope_sin + rope_tab * p.rope_table_stride : nullptr;
    const int kv_len = valid_len<MASK>(p.n_k, p.ctx_keys);
    const int last = p.n_k - 1;

    // ---- stage K, V, key terms, T5 table and q: every load is issued before the first wait ----
    f32x4 klo[RKIT], khi[RKIT], kcs[RKIT], ksn[RKIT];
#pragma unroll
    for (int u = 0; u < RKIT; u++) {  // K item = (row, c): dims 4c..4c+3 and 32+4c..32+4c+3
        const int it = tid + u * RNT, row = it >> 3, c = it & 7, rc = min(row, last);
        const float* src = K + (int64_t)rc * p.k_tok + 4 * c;
        klo[u] = ld4(src);
        khi[u] = ld4(src + 32);
        if (ROPE) {
            kcs[u] = ld4(RC + (int64_t)rc * 32 + 4 * c);
            ksn[u] = ld4(RS + (int64_t)rc * 32 + 4 * c);
        }
    }
    f32x4 v01[RVIT], v23[RVIT];
#pragma unroll
    for (int u = 0; u < RVIT; u++) {  // V item = (quad of 4 rows, dims 2vc, 2vc+1)
        const int it = tid + u * RNT, quad = it >> 5, vc = it & 31, r0 = 4 * quad;
        const float* src = V + 2 * vc;
        const f32x2 a = ld2(src + (int64_t)min(r0, last) * p.v_tok);
        const f32x2 bb = ld2(src + (int64_t)min(r0 + 1, last) * p.v_tok);
        const f32x2 c = ld2(src + (int64_t)min(r0 + 2, last) * p.v_tok);
        const f32x2 d = ld2(src + (int64_t)min(r0 + 3, last) * p.v_tok);
        v01[u] = f32x4{r0 <= last ? a[0] : 0.f, r0 <= last ? a[1] : 0.f, r0 + 1 <= last ? bb[0] : 0.f,
                       r0 + 1 <= last ? bb[1] : 0.f};
        v23[u] = f32x4{r0 + 2 <= last ? c[0] : 0.f, r0 + 2 <= last ? c[1] : 0.f, r0 + 3 <= last ? d[0] : 0.f,
                       r0 + 3 <= last ? d[1] : 0.f};
    }
    float kterm = 0.f;
    if (tid < lay.nkp) {
        bool valid = true;
        if (mask_reads_valid<MASK>()) valid = tid < kv_len && KV[tid] != 0;
        kterm = key_term<MASK>(tid, p.n_k, valid, p.ctx_keys);
    }
    float qreg[RQB][16];
#pragma unroll
    for (int qb = 0; qb < RQB; qb++) {
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
                rope4(a0, a2, ld4(RC + row + 8 * g), ld4(RS + row + 8 * g));
                rope4(a1, a3, ld4(RC + row + 8 * g + 4), ld4(RS + row + 8 * g + 4));
            }
            a0 *= p.scale;  // power-of-two scales: exact, as in the streaming kernel
            a1 *= p.scale;
            a2 *= p.scale;
            a3 *= p.scale;
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            qreg[qb][t] = a0[t];
            qreg[qb][4 + t] = a1[t];
            qreg[qb][8 + t] = a2[t];
            qreg[qb][12 + t] = a3[t];
        }
    }
    if (BIAS == BIAS_REL) {
        const int n_rel = p.n_q + p.n_k - 1;
        for (int t0 = 0; t0 < n_rel; t0 += 2 * RNT) {
            const int t1 = t0 + tid, t2 = t1 + RNT;
            const int b1 = t1 < n_rel ? min(max(p.rel_bucket[t1], 0), p.rel_buckets - 1) : 0;
            const int b2 = t2 < n_rel ? min(max(p.rel_bucket[t2], 0), p.rel_buckets - 1) : 0;
            const float x1 = p.rel_table[b1 * p.H + h], x2 = p.rel_table[b2 * p.H + h];
            if (t1 < n_rel) lut[t1] = x1;
            if (t2 < n_rel) lut[t2] = x2;
        }
    }
#pragma unroll
    for (int u = 0; u < RKIT; u++) {
        const int it = tid + u * RNT, row = it >> 3, c = it & 7;
        if (row >= lay.nkp) continue;
        f32x4 lo = row <= last ? klo[u] : f32x4{0, 0, 0, 0}, hi = row <= last ? khi[u] : f32x4{0, 0, 0, 0};
        if (ROPE) rope4(lo, hi, kcs[u], ksn[u]);
        st4(Ks + row * KPAD + 4 * c, lo);
        st4(Ks + row * KPAD + 32 + 4 * c, hi);
    }
#pragma unroll
    for (int u = 0; u < RVIT; u++) {
        const int it = tid + u * RNT, quad = it >> 5, vc = it & 31;
        if (4 * quad >= lay.nkp) continue;
        float* vd = Vs + quad * (kHeadDim * 4);
        st4(vd + vslot(2 * vc) * 4, f32x4{v01[u][0], v01[u][2], v23[u][0], v23[u][2]});
        st4(vd + vslot(2 * vc + 1) * 4, f32x4{v01[u][1], v01[u][3], v23[u][1], v23[u][3]});
    }
    if (tid < lay.nkp) kadd[tid] = kterm;
    __syncthreads();  // the only barrier: everything below reads LDS that no one writes again

    const int wave_nq = max(0, min(16 * RQB, p.n_q - wq0));
    if (wave_nq == 0) return;
    const int nqb = (wave_nq + 15) >> 4;
    const int wave_kend = key_end_for<MASK>(p.q_pos0 + wq0 + wave_nq - 1, p.n_k, p.ctx_keys);
    const int voff_even = vslot(ql) * 4, voff_odd = vslot(16 + ql) * 4;

    float m_run[RQB], ml_run[RQB], l_run[RQB];
    f32x4 oacc[4][RQB];
#pragma unroll
    for (int qb = 0; qb < RQB; qb++) {
        m_run[qb] = ml_run[qb] = kNegInf;
        l_run[qb] = 0.f;
#pragma unroll
        for (int db = 0; db < 4; db++) oacc[db][qb] = f32x4{0, 0, 0, 0};
    }

    auto tile = [&](int kbase, int nkb, auto plain_tag) {
        constexpr bool PLAIN = decltype(plain_tag)::value;
        f32x4 sacc[4][RQB];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
#pragma unroll
            for (int qb = 0; qb < RQB; qb++) sacc[kb][qb] = f32x4{0, 0, 0, 0};
            if (!PLAIN && kb >= nkb) continue;
            const float* kr = Ks + (kbase + kb * 16 + ql) * KPAD;
            const f32x4 k0 = ld4(kr + 8 * g), k1 = ld4(kr + 8 * g + 4);
            const f32x4 k2 = ld4(kr + 32 + 8 * g), k3 = ld4(kr + 32 + 8 * g + 4);
            const float kv16[16] = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3],
                                    k2[0], k2[1], k2[2], k2[3], k3[0], k3[1], k3[2], k3[3]};
#pragma unroll
            for (int qb = 0; qb < RQB; qb++) {
                if (!PLAIN && qb >= nqb) continue;
                f32x4 c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
#pragma unroll
                for (int s = 0; s < 16; s += 4) {
                    c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv16[s], qreg[qb][s], c0, 0, 0, 0);
                    c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv16[s + 1], qreg[qb][s + 1], c1, 0, 0, 0);
                    c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv16[s + 2], qreg[qb][s + 2], c2, 0, 0, 0);
                    c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv16[s + 3], qreg[qb][s + 3], c3, 0, 0, 0);
                }
                sacc[kb][qb] = (c0 + c1) + (c2 + c3);
                asm volatile("" : "+v"(sacc[kb][qb]));  // keep the tree sum here (see above)
            }
        }
#pragma unroll
        for (int qb = 0; qb < RQB; qb++) {
#pragma clang fp contract(off)
            if (!PLAIN && qb >= nqb) continue;
            const int qi = wq0 + 16 * qb + ql;
            const int qpos = p.q_pos0 + qi;
            float mloc = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const bool on = PLAIN || kb < nkb;
                f32x4 ka = {0, 0, 0, 0};
                if (!PLAIN && on) ka = ld4(kadd + kbase + kb * 16 + 4 * g);  // blocks past nkb: past nkp
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = kbase + kb * 16 + 4 * g + r;
                    float x = kNegInf;
                    if (on) {
                        x = sacc[kb][qb][r];
                        if (BIAS == BIAS_REL) x = x + lut[min(max(key - qi + p.n_q - 1, 0), p.n_q + p.n_k - 2)];
                        if (BIAS == BIAS_DENSE && (PLAIN || (key < p.n_k && qi < p.n_q)))
                            x = x + p.bias[h * p.bias_head + (int64_t)qi * p.bias_row + key];
                        if (!PLAIN) x = masked<MASK>(x, ka[r], key, qpos, p.n_k, p.chain_start);
                    }
                    sacc[kb][qb][r] = x;
                    mloc = fmaxf(mloc, x);
                }
            }
            const float m_new = fmaxf(m_run[qb], max4(mloc));
            const float m_use = m_new == kNegInf ? 0.f : m_new;
            float alpha, lsum = 0.f;
            if (__ballot(m_use < -1e30f) == 0) {
                const float ml = m_use * kLog2e;
                alpha = __builtin_amdgcn_exp2f(ml_run[qb] - ml);
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][qb][r], kLog2e, -ml));
                        sacc[kb][qb][r] = e;
                        lsum += e;
                    }
                ml_run[qb] = m_new == kNegInf ? kNegInf : ml;
            } else {
                alpha = __builtin_amdgcn_exp2f((m_run[qb] - m_use) * kLog2e);
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float e = __builtin_amdgcn_exp2f((sacc[kb][qb][r] - m_use) * kLog2e);
                        sacc[kb][qb][r] = e;
                        lsum += e;
                    }
                ml_run[qb] = m_new == kNegInf ? kNegInf : m_use * kLog2e;
            }
            l_run[qb] = l_run[qb] * alpha + lsum;
            m_run[qb] = m_new;
            if (__ballot(alpha != 1.f) != 0) {
#pragma unroll
                for (int db = 0; db < 4; db++) oacc[db][qb] *= alpha;
            }
        }
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            if (!PLAIN && kb >= nkb) continue;
            const float* vq4 = Vs + ((kbase >> 2) + kb * 4 + g) * (kHeadDim * 4);
            f32x4 va[4];
#pragma unroll
            for (int db = 0; db < 4; db++) va[db] = ld4(vq4 + db * 64 + ((db & 1) ? voff_odd - 64 : voff_even));
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int db = 0; db < 4; db++)
#pragma unroll
                    for (int qb = 0; qb < RQB; qb++) {
                        if (!PLAIN && qb >= nqb) continue;
                        oacc[db][qb] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[db][r], sacc[kb][qb][r], oacc[db][qb], 0, 0, 0);
                    }
        }
    };

    for (int kbase = 0; kbase < wave_kend; kbase += NK) {
        const int nkb = min(4, (wave_kend - kbase + 15) >> 4);
        bool plain = kbase + NK <= wave_kend && wave_nq == 16 * RQB && MASK != DECODER;
        if (plain && mask_reads_valid<MASK>()) plain = __ballot(kadd[kbase + lane] != 0.f) == 0;
        if (MASK == CAUSAL || MASK == CAUSAL_KEYS) plain = plain && kbase + NK - 1 <= p.q_pos0 + wq0;
        if (plain) tile(kbase, 4, std::integral_constant<bool, true>{});
        else tile(kbase, nkb, std::integral_constant<bool, false>{});
    }

#pragma unroll
    for (int qb = 0; qb < RQB; qb++) {
        const int qi = wq0 + 16 * qb + ql;
        const float l = sum4(l_run[qb]);
        if (qi >= p.n_q) continue;
        const float inv = 1.0f / l;
        float* dst = O + (int64_t)qi * p.o_tok;
#pragma unroll
        for (int db = 0; db < 4; db++) st4(dst + 16 * db + 4 * g, oacc[db][qb] * inv);
    }
}

template <int MASK, int BIAS, bool ROPE>
hipError_t launch_one(const Params& p, hipStream_t stream) {
    if (p.n_k <= kResidentKeys) {  // short rows: the whole K/V of a (series, head) in LDS
        const int q_tiles = (p.n_q + RQT - 1) / RQT;
        const int64_t blocks = (int64_t)p.B * p.H * q_tiles;
        if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
        const size_t lds = (size_t)resident_layout(p.n_q, p.n_k, BIAS == BIAS_REL).total * sizeof(float);
        hipLaunchKernelGGL((attn_fwd_f32_resident<MASK, BIAS, ROPE>), dim3((unsigned)blocks), dim3(RNT), lds, stream,
                           p);
        return hipGetLastError();
    }
    const int q_tiles = (p.n_q + QT - 1) / QT;
    const int64_t blocks = (int64_t)p.B * p.H * q_tiles;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fwd_f32<MASK, BIAS, ROPE>), dim3((unsigned)blocks), dim3(NT), 0, stream, p);
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
