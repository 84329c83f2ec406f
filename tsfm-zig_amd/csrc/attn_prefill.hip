// Pipelined bf16 / f16 attention with f32 accumulation for gfx950, for the masks whose excluded
// keys carry -inf (FULL, CAUSAL, CAUSAL_KEYS, FULL_KEYS) without RoPE: Timestral's causal prefill
// (src/timestral/model.zig:580-635, selfAttend at src/core/attn.zig:72-96) and any other
// half-precision call of those masks. One workgroup = one (series, head) x 128 queries, 4 waves x
// 32 queries, 64-key tiles, on v_mfma_f32_32x32x16_{f16,bf16}.
//
//   S^T = K . Q^T   per 32-key block: A = 32 K rows x 16 dims (lane: key l%32, dims 8(l/32)..+7),
//                   B = Q^T (lane: query l%32), four instructions over the 64 head dims. The
//                   accumulator lane l holds query l%32 and keys 8(r/4) + 4(l/32) + r%4, r < 16.
//   O^T += V^T . P^T  per 16-key chunk: B = P^T packed from eight S^T registers of the lane
//                   (k-slot 8(l/32)+j <-> key 4(l/32) + j for j < 4, 8 + 4(l/32) + j-4 for j >= 4),
//                   A = V^T read from LDS with the transposing ds_read_b64_tr_b16 in that same key
//                   order; two instructions (32 dims each) per chunk.
//
// Software pipeline per wave, over 32-key blocks: block j+1's S^T chain is issued on the matrix
// cores inside the same straight-line region as block j's exponentials on the VALU (one quarter of
// the exponentials between consecutive matrix instructions), then block j's P.V products; the
// matrix work of one block overlaps the softmax of the previous one instead of waiting for it.
// Staging: K and V tiles go from HBM / L2 straight into LDS (buffer_load_dwordx4 ... lds through
// buffer descriptors whose range ends after the last key, so a ragged tail reads zeros), K two
// tiles ahead in the operand order of the S^T instruction (each operand read is 1 KB of contiguous
// LDS), V one tile ahead as rows with their 16-byte chunks XOR-swizzled by key (conflict-free
// transposing reads). No staging registers, one barrier per tile.
//
// Softmax in f32 registers, in exp2 units: e = exp2(s * scale*log2(e) - m). A block's weights are
// formed against the current m first; m moves only when they show it must (a lane's rounded
// weights sum past 2^8, or a row's sum is below 1/2: its max is not established), so m may trail
// the true max by up to 8 and the check reads only VALU results. The row sum is taken over the
// weights rounded to the input type (the weights the P.V product applies), with v_dot2 on the
// VALU. Excluded keys give exactly 0.
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(3))) i16x4* lds_i16x4_ptr;

constexpr int QW = 32;                 // queries per wave
constexpr int NWAVE = 4;
constexpr int NT = 64 * NWAVE;
constexpr int QT = QW * NWAVE;         // queries per workgroup
constexpr int NK = 64;                 // keys per tile
constexpr int kChunk = 8;             // (series, head) pairs per chunk of causal work-groups
constexpr int STAGE = NK * kHeadDim / 2;  // dwords per K or V stage (8 KB)
constexpr float kStaleSum = 256.f;  // 2^8: the largest sum of a lane's 16 weights that leaves the max
#ifndef WAVES_PER_SIMD
#define WAVES_PER_SIMD 4
#endif

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
}

// Sum of the two rounded weights of a packed pair, added to acc (v_dot2 with (1, 1)).
template <bool BF16>
__device__ __forceinline__ float dot2_ones(uint32_t w, float acc) {
    if constexpr (BF16) {
        const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
    } else {
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, acc, false);
    }
}

__device__ __forceinline__ u32x4 ldu4(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Position of the 16-byte chunk c of a V row in LDS: chunks XOR-swizzled by the key's row. A
// transposing read takes 32 bytes (two chunks, one pair index) from each of four consecutive rows per
// 16-lane group; XOR-ing the pair index with the row's low two bits puts the four rows on four
// different 32-byte bank ranges, so a group covers all 32 banks once.
__device__ __forceinline__ int vchunk(int key_local, int c) { return c ^ ((key_local & 3) << 1); }

// LDS: three K stages, then two V stages, 8 KB each.
constexpr uint32_t kStageBytes = STAGE * 4;
constexpr uint32_t kVBase = 3 * kStageBytes;
typedef __attribute__((address_space(3))) u32x4* lds_u32x4_ptr;
__device__ __forceinline__ u32x4 lds_read16(uint32_t addr) { return *(lds_u32x4_ptr)(uintptr_t)addr; }

__device__ __forceinline__ u32x2 lds_read_tr(uint32_t addr) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_ptr)(uintptr_t)addr));
}

template <bool BF16, int MASK>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(WAVES_PER_SIMD, WAVES_PER_SIMD))) void
attn_fwd_half_pipe(Params p) {
    __shared__ __attribute__((aligned(1024))) uint32_t smem[5 * STAGE];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t*)smem;

    typedef uint16_t E;
    constexpr bool kCausal = MASK == CAUSAL || MASK == CAUSAL_KEYS;
    constexpr bool kValid = MASK == CAUSAL_KEYS || MASK == FULL_KEYS;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: wave-level decisions branch on SGPRs
    const int lq = lane & 31, lh = lane >> 5;
    const int q_tiles = (p.n_q + QT - 1) / QT;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    int bh = logical / q_tiles, qt = logical % q_tiles;
    if (kCausal) {
        // Causal tiles differ in length (tile qt reads qt + 1 key tiles). Consecutive work-groups
        // (one XCD's, in dispatch order) take chunks of kChunk (series, head) pairs, and within a
        // chunk all its pairs' longest tiles come first: the XCD's resident work-groups share the
        // K/V of a few pairs in its L2, and the short tiles fill in behind the long ones instead
        // of a long tile starting last.
        const int nbh = p.B * p.H, span = kChunk * q_tiles;
        const int chunk = logical / span, r = logical - chunk * span;
        const int cs = min(kChunk, nbh - chunk * kChunk);
        qt = q_tiles - 1 - r / cs;
        bh = chunk * kChunk + r % cs;
    }
    const int b = bh / p.H, h = bh % p.H;
    const int q0 = qt * QT, wq0 = q0 + wave * QW;

    const E* __restrict__ Q = static_cast<const E*>(p.q) + b * p.q_batch + h * kHeadDim;
    const E* __restrict__ K = static_cast<const E*>(p.k) + b * p.k_batch + h * kHeadDim;
    const E* __restrict__ V = static_cast<const E*>(p.v) + b * p.v_batch + h * kHeadDim;
    E* __restrict__ O = static_cast<E*>(p.o) + b * p.o_batch + h * kHeadDim;
    const uint8_t* __restrict__ KV = kValid ? p.key_valid + b * p.kv_batch : nullptr;

    const int wg_qhi = p.q_pos0 + min(p.n_q, q0 + QT) - 1;
    const int kend = key_end_for<MASK>(wg_qhi, p.n_k, 0);
    const int ntiles = (kend + NK - 1) / NK;
    const int wave_nq = max(0, min(QW, p.n_q - wq0));
    const int wave_qlo = p.q_pos0 + wq0;
    const int wave_kend = wave_nq > 0 ? key_end_for<MASK>(wave_qlo + wave_nq - 1, p.n_k, 0) : 0;
    const int qpos = wave_qlo + lq;
    const float c2 = p.scale * kLog2e;  // > 0 (checked on the host)

    // Q^T operand per 16-dim step s: query wq0 + l%32, dims 16s + 8(l/32) .. +7.
    u32x4 qf[4];
    {
        const int qi = wq0 + lq;
#pragma unroll
        for (int s = 0; s < 4; s++)
            qf[s] = qi < p.n_q ? ldu4(Q + (int64_t)qi * p.q_tok + 16 * s + 8 * lh) : u32x4{0, 0, 0, 0};
    }

    // ---- staging: each wave moves two 1 KB blocks of K and two of V per tile ----
    // K block (kb, s) of a stage (kb = key block of 32, s = 16-dim step) holds, at 16 l, lane l's
    // operand of the S^T instruction: key 32 kb + l%32, dims 16 s + 8 (l/32) .. +7. V rows are 128
    // bytes, key-major, chunk c of row kl at 16-byte slot vchunk(kl, c). Loads go through buffer
    // descriptors that end after key n_k - 1, so rows past it read as zeros (weight 0 keys) without
    // a clamp; a lane's byte offset within a tile is fixed, the tile adds kbase rows as a scalar
    // offset (the host keeps a (series, head) span of K or V below 4 GiB).
    const u32x4 k_buf = buf_desc(K, (uint32_t)(((int64_t)(p.n_k - 1) * p.k_tok + kHeadDim) * 2));
    const u32x4 v_buf = buf_desc(V, (uint32_t)(((int64_t)(p.n_k - 1) * p.v_tok + kHeadDim) * 2));
    uint32_t k_off[2], v_off[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int blk = 2 * wave + i, kb = blk >> 2, s = blk & 3;
        k_off[i] = (uint32_t)((32 * kb + lq) * p.k_tok + 16 * s + 8 * lh) * 2u;
        const int kl = 8 * blk + (lane >> 3);
        v_off[i] = (uint32_t)(kl * p.v_tok + 8 * vchunk(kl, lane & 7)) * 2u;  // the chunk for slot lane % 8
    }
    auto stage_k = [&](int t) {
        const uint32_t st = lds0 + (uint32_t)(t % 3) * kStageBytes + (uint32_t)wave * 2048u;
        const uint32_t so = (uint32_t)(t * NK) * (uint32_t)p.k_tok * 2u;
#pragma unroll
        for (int i = 0; i < 2; i++) dma16(k_buf, st + i * 1024u, k_off[i], so);
    };
    auto stage_v = [&](int t) {
        const uint32_t st = lds0 + kVBase + (uint32_t)(t & 1) * kStageBytes + (uint32_t)wave * 2048u;
        const uint32_t so = (uint32_t)(t * NK) * (uint32_t)p.v_tok * 2u;
#pragma unroll
        for (int i = 0; i < 2; i++) dma16(v_buf, st + i * 1024u, v_off[i], so);
    };
    // key_valid byte of key t*NK + lane (0 past the bytes the mask reads).
    auto kv_byte = [&](int t) -> uint32_t {
        if (!kValid) return 1u;
        const int key = t * NK + lane;
        return key < p.n_k ? (uint32_t)KV[key] : 0u;
    };

    // The pipeline runs over 32-key blocks: block j is key block j%2 of tile j/2. S^T of block j
    // from K stage (j/2) % 3: one chain of four instructions over the 64 head dims.
    const uint32_t k_lane = lane * 16u;
    auto scores = [&](int j, f32x16& sb) {
        const uint32_t kr = lds0 + (uint32_t)((j >> 1) % 3) * kStageBytes + (uint32_t)(j & 1) * 4096u + k_lane;
        sb = mfma32<BF16>(lds_read16(kr), qf[0], f32x16{});
#pragma unroll
        for (int s = 1; s < 4; s++) sb = mfma32<BF16>(lds_read16(kr + s * 1024u), qf[s], sb);
    };

    f32x16 oacc[2] = {f32x16{}, f32x16{}};
    float m_use = 0.f;  // the max (exp2 units) every accumulated weight is taken against
    float lsum = 0.f;

    // Transposing V reads: lane l, read rho of chunk c and dim block db gets dim 32 db + l%32 of the
    // keys 16 c + 4 (l/32) + 8 rho + j (j < 4). The source address of lane l (group g = l/16, s = l%16)
    // is key 16 c + 4 (g/2) + 8 rho + s/4, dims 32 db + 16 (g%2) + 4 (s%4) .. +3; the key's row
    // offset within its 8-row group, and so its swizzle, is the same for every (c, rho).
    const int tr_key = 4 * (lane >> 5) + ((lane & 15) >> 2);
    const int tr_dim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    uint32_t v_lane[2];
#pragma unroll
    for (int db = 0; db < 2; db++) {
        const int dim = 32 * db + tr_dim;
        v_lane[db] = (uint32_t)(tr_key * 128 + vchunk(tr_key, dim >> 3) * 16 + ((dim >> 2) & 1) * 8);
    }
    auto v_operand = [&](uint32_t vs, int db, int c) -> u32x4 {
        const uint32_t a = vs + v_lane[db] + (uint32_t)(16 * c) * 128u;
        const u32x2 lo = lds_read_tr(a), hi = lds_read_tr(a + 8u * 128u);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };

    // Block j's flags for this wave, from its tile's validity ballot vm (bits = keys of the tile).
    auto block_bits = [](int j, uint64_t vm) { return (uint32_t)(vm >> (32 * (j & 1))); };
    auto is_plain = [&](int j, uint64_t vm) {
        const int k0 = j * 32;
        bool pl = k0 + 32 <= p.n_k;
        if (kValid) pl = pl && block_bits(j, vm) == ~0u;
        if (kCausal) pl = pl && k0 + 31 <= wave_qlo;
        return pl;
    };
    auto is_active = [&](int j, uint64_t vm) {
        const int k0 = j * 32;
        if (k0 >= wave_kend) return false;
        if (!kValid) return true;
        const bool diag = k0 < wave_qlo + QW && k0 + 32 > wave_qlo;  // an always-open diagonal key
        return block_bits(j, vm) != 0 || diag;
    };

    // Block j's mask on the raw scores (blocks that are not mask-free). Register r holds key
    // offset 4 (l/32) + o(r) in the block, o(r) = 8 (r/4) + r%4. The lane's allowed registers are
    // formed as one 16-bit word, then applied: excluded keys become -inf.
    auto mask_scores = [&](int j, f32x16& sb, uint64_t vm) {
        // Registers r with o(r) <= d: the low n(d) bits (o is increasing in r).
        auto upto = [](int d) -> uint32_t {
            const int n = d < 0 ? 0 : d >= 27 ? 16 : 4 * (d >> 3) + min(4, (d & 7) + 1);
            return (1u << n) - 1u;
        };
        const int base = j * 32 + 4 * lh;  // key of o = 0
        uint32_t a = upto(p.n_k - 1 - base);  // in range
        if (MASK == CAUSAL) a &= upto(qpos - base);
        if (kValid) {
            const uint32_t x = block_bits(j, vm) >> (4 * lh);  // bit o = key base + o valid
            const uint32_t valid = (x & 0xfu) | ((x >> 4) & 0xf0u) | ((x >> 8) & 0xf00u) | ((x >> 12) & 0xf000u);
            const int dd = qpos - base;  // the diagonal's o, when it is one of the lane's
            const uint32_t diag = (dd >= 0 && dd < 32 && (dd & 7) < 4) ? 1u << (4 * (dd >> 3) + (dd & 7)) : 0u;
            if (MASK == CAUSAL_KEYS) a &= (valid & upto(dd)) | diag;
            else a &= valid | diag;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) sb[r] = (a >> r) & 1u ? sb[r] : kNegInf;
    };
    // Quarter q of a block's weights (registers 4q .. 4q+3): two packed pairs into pf[q/2], and
    // their rounded sum into ls[q%2].
    auto weights_part = [&](const f32x16& sb, int q, u32x4 (&pf)[2], float (&ls)[2]) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sb[4 * q], c2, -m_use));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sb[4 * q + 1], c2, -m_use));
        const float e2 = __builtin_amdgcn_exp2f(__builtin_fmaf(sb[4 * q + 2], c2, -m_use));
        const float e3 = __builtin_amdgcn_exp2f(__builtin_fmaf(sb[4 * q + 3], c2, -m_use));
        const uint32_t w0 = pack2<BF16>(e0, e1), w1 = pack2<BF16>(e2, e3);
        pf[q >> 1][2 * (q & 1)] = w0;
        pf[q >> 1][2 * (q & 1) + 1] = w1;
        ls[q & 1] = dot2_ones<BF16>(w1, dot2_ones<BF16>(w0, ls[q & 1]));
    };
    // O^T += V^T P^T over block j's two 16-key chunks, V from stage (j/2) & 1. All eight
    // transposing reads (two chunks x two 32-dim blocks) are issued before the first instruction.
    auto pv = [&](int j, const u32x4 (&pf)[2]) {
        const uint32_t vs = lds0 + kVBase + (uint32_t)((j >> 1) & 1) * kStageBytes;
        u32x4 va[2][2];
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int db = 0; db < 2; db++) va[c][db] = v_operand(vs, db, 2 * (j & 1) + c);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int db = 0; db < 2; db++) oacc[db] = mfma32<BF16>(va[c][db], pf[c], oacc[db]);
    };
    // The weights of a block are formed against the current m_use first; the max moves only when
    // they show it must: some lane's rounded weights sum past kStaleSum (a weight past it), or a
    // row's accumulated sum is below 1/2 (its max is not established: m_use starts at 0; once it is,
    // the max's own weight keeps the sum at 1 or more). Then
    // the row max over both lanes of each query (l and l ^ 32) becomes m_use (for a row below 1/2
    // it may move down; otherwise only up), O and the row sum are rescaled, and the block's weights are
    // formed again. The check reads only the block's own VALU results, not the matrix cores'.
    auto check_update = [&](const f32x16& sb, u32x4 (&pf)[2], float& ls) {
        const float tot = lsum + ls;
        const auto st = __builtin_amdgcn_permlane32_swap(__float_as_uint(tot), __float_as_uint(tot), false, false);
        const float row = __uint_as_float(st[0]) + __uint_as_float(st[1]);
        if (__ballot(ls > kStaleSum || row < 0.5f) == 0) return;
        float m = sb[0];
#pragma unroll
        for (int r = 1; r < 16; r++) m = fmaxf(m, sb[r]);
        const float mt = m * c2;  // exp2 units (the scale is positive)
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
        const float mk = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        if (mk != kNegInf) {  // a query with no score in this block keeps its state
            const float mn = row < 0.5f ? mk : fmaxf(m_use, mk);
            // O and lsum hold weights against m_use; a row below 1 may scale up (capped: a row
            // with nothing accumulated scales zeros).
            const float alpha = fminf(__builtin_amdgcn_exp2f(m_use - mn), 0x1p64f);
#pragma unroll
            for (int db = 0; db < 2; db++) oacc[db] *= alpha;
            lsum *= alpha;
            m_use = mn;
        }
        float lp[2] = {0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 4; q++) weights_part(sb, q, pf, lp);
        ls = lp[0] + lp[1];
    };

    const int nblocks = 2 * ntiles;
    uint64_t vm0 = 0, vm1 = 0;  // validity ballots of tiles t and t+1
    bool act = false;           // the wave has block j
    // Block j with its scores in cur (raw): its mask when it is not mask-free; block j+1's S^T on
    // the matrix cores in the same straight-line region as block j's exponentials on the VALU; the
    // max check; block j's P.V. vmc / vmn: the ballots of
    // block j's and block j+1's tiles.
    auto block = [&](int j, f32x16& cur, f32x16& nxt, uint64_t vmc, uint64_t vmn) {
        const bool act1 = j + 1 < nblocks && is_active(j + 1, vmn);
        u32x4 pf[2];
        float ls = 0.f;
        if (act && !is_plain(j, vmc)) mask_scores(j, cur, vmc);
        if (act && act1) {
            // Written in issue order, fenced so the scheduler keeps it: a quarter of block j's
            // exponentials between consecutive matrix instructions of block j+1's S^T chain, each
            // K operand read one instruction ahead of its use.
            const uint32_t kr = lds0 + (uint32_t)(((j + 1) >> 1) % 3) * kStageBytes + (uint32_t)((j + 1) & 1) * 4096u +
                                k_lane;
            u32x4 ka = lds_read16(kr), kb = lds_read16(kr + 1024u);
            float lp[2] = {0.f, 0.f};
            __builtin_amdgcn_sched_barrier(0);
            weights_part(cur, 0, pf, lp);
            __builtin_amdgcn_sched_barrier(0);
            nxt = mfma32<BF16>(ka, qf[0], f32x16{});
            ka = lds_read16(kr + 2048u);
            __builtin_amdgcn_sched_barrier(0);
            weights_part(cur, 1, pf, lp);
            __builtin_amdgcn_sched_barrier(0);
            nxt = mfma32<BF16>(kb, qf[1], nxt);
            kb = lds_read16(kr + 3072u);
            __builtin_amdgcn_sched_barrier(0);
            weights_part(cur, 2, pf, lp);
            __builtin_amdgcn_sched_barrier(0);
            nxt = mfma32<BF16>(ka, qf[2], nxt);
            __builtin_amdgcn_sched_barrier(0);
            weights_part(cur, 3, pf, lp);
            __builtin_amdgcn_sched_barrier(0);
            nxt = mfma32<BF16>(kb, qf[3], nxt);
            __builtin_amdgcn_sched_barrier(0);
            ls = lp[0] + lp[1];
        } else if (act) {
            float lp[2] = {0.f, 0.f};
#pragma unroll
            for (int q = 0; q < 4; q++) weights_part(cur, q, pf, lp);
            ls = lp[0] + lp[1];
        } else if (act1) {
            scores(j + 1, nxt);
        }
        if (act) {
            check_update(cur, pf, ls);
            lsum += ls;
            pv(j, pf);
        }
        act = act1;
    };

    // ---- prologue: tiles 0 and 1 of K, tile 0 of V, the validity of tiles 0 and 1 ----
    {
        const uint32_t kb0 = ntiles > 0 ? kv_byte(0) : 0u, kb1 = ntiles > 1 ? kv_byte(1) : 0u;
        if (ntiles > 0) {
            stage_k(0);
            stage_v(0);
        }
        if (ntiles > 1) stage_k(1);
        vm0 = __ballot(kb0 != 0);
        vm1 = __ballot(kb1 != 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // Q has landed on every path: an empty use in registers here, so the compiler puts no wait for
    // it inside the loop (where a wait for global loads would also wait for the staging).
    asm volatile("" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]));

    f32x16 sa, sb;
    act = ntiles > 0 && is_active(0, vm0);
    if (act) scores(0, sa);
    // One tile (two blocks) per iteration, so the score buffers trade roles without copies; the
    // staging of tiles t+1 (V) and t+2 (K) is issued first and published by the barrier at the end.
    for (int t = 0; t < ntiles; t++) {
        const bool more1 = t + 1 < ntiles, more2 = t + 2 < ntiles;
        const uint32_t kb2 = more2 ? kv_byte(t + 2) : 0u;
        if (more2) stage_k(t + 2);
        if (more1) stage_v(t + 1);
        __builtin_amdgcn_sched_barrier(0);
        block(2 * t, sa, sb, vm0, vm0);
        block(2 * t + 1, sb, sa, vm0, vm1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        vm0 = vm1;
        vm1 = __ballot(kb2 != 0);
    }

    // ---- normalise and store: lane holds query wq0 + l%32, dims 32 db + 8 a + 4 (l/32) .. +3 ----
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum), __float_as_uint(lsum), false, false);
    const float l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    const int qi = wq0 + lq;
    if (qi < p.n_q) {
        const float inv = 1.0f / l;
        E* dst = O + (int64_t)qi * p.o_tok + 4 * lh;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const f32x4 o = {oacc[db][4 * a] * inv, oacc[db][4 * a + 1] * inv, oacc[db][4 * a + 2] * inv,
                                 oacc[db][4 * a + 3] * inv};
                *reinterpret_cast<u32x2*>(dst + 32 * db + 8 * a) = u32x2{pack2<BF16>(o[0], o[1]), pack2<BF16>(o[2], o[3])};
            }
    }
}

template <bool BF16, int MASK>
hipError_t launch_one(const Params& p, hipStream_t stream) {
    const int q_tiles = (p.n_q + QT - 1) / QT;
    const int64_t blocks = (int64_t)p.B * p.H * q_tiles;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL((attn_fwd_half_pipe<BF16, MASK>), dim3((unsigned)blocks), dim3(NT), 0, stream, p);
    return hipGetLastError();
}

template <bool BF16>
hipError_t launch_mask(const Params& p, int mask, hipStream_t s) {
    switch (mask) {
    case FULL: return launch_one<BF16, FULL>(p, s);
    case CAUSAL: return launch_one<BF16, CAUSAL>(p, s);
    case CAUSAL_KEYS: return launch_one<BF16, CAUSAL_KEYS>(p, s);
    case FULL_KEYS: return launch_one<BF16, FULL_KEYS>(p, s);
    default: return hipErrorNotSupported;
    }
}

}  // namespace

bool attn_half_pipe_supports(const Params& p, int mask, int bias, bool rope) {
    if (rope || bias != BIAS_NONE || !(p.scale > 0.f)) return false;
    if (mask != FULL && mask != CAUSAL && mask != CAUSAL_KEYS && mask != FULL_KEYS) return false;
    return p.n_k > 0;
}

hipError_t launch_attn_half_pipe(const Params& p, bool is_bf16, int mask, hipStream_t s) {
    return is_bf16 ? launch_mask<true>(p, mask, s) : launch_mask<false>(p, mask, s);
}

}  // namespace tsfm
