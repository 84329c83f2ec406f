// Fused Q/K/V (and gate) projection with rotate-half RoPE in the epilogue, f32 on the matrix cores
// (gfx950).
//
// What it replaces, for the time-attention block of each family:
//  - Chronos-2: three nn.linear calls (q, k, v) and the serial RoPE loop over every (token, head)
//    (src/chronos2/model.zig:232-245);
//  - Timestral: the fused qkv nn.linear over the permuted (qkv, head, head_dim) weight, the gate
//    nn.linear, and TimeJob.rope (src/timestral/model.zig:495,500,513,558-577); without RoPE,
//    the projections of Model.variateAttention (:532,535);
//  - Chronos-Bolt: the q, k, v nn.linear calls of the encoder self-attention
//    (src/chronos_bolt/model.zig:239-241, no RoPE).
// nn.linear (src/core/nn.zig:262-293) is y[rows, out] = x[rows, in] w[out, in]^T; these calls pass
// no bias. RoPE is nn.ropeHalf (src/core/nn.zig:448-467) on each 64-wide head of q and k.
//
// One launch computes every output: the output columns are the concatenation [q | k | v | gate]
// (each heads * 64 wide), so x is streamed through the chip once for all of them. A workgroup
// computes a token x column tile, K = d_in in 16- or 32-wide steps: x and w tiles go from HBM/L2
// straight into LDS (global_load_lds_dwordx4, double-buffered, one barrier per step), laid out in
// the order the operand reads take them (no bank conflicts, no staging registers), and each wave
// multiplies a 32-token sub-tile with v_mfma_f32_16x16x4_f32, the weight rows as the A operand so
// that each lane ends with four consecutive output columns of one token (16-byte stores, and the
// RoPE partner column i + 32 in the same lane); f32 outputs, or bf16/f16 for the half-precision
// attention path. Large products take 128 x 128 tiles (8 waves of 32 tokens x one 64-column head,
// two workgroups per CU; the tokens of a last round of tiles that would leave most CUs idle go to
// a second launch of small tiles); small ones, and those whose reduction is split over
// workgroups, 64 x 64 tiles (4 waves of 32 x 32, four workgroups per CU).
//
// Accumulation order. v_mfma_f32_16x16x4_f32 rounds as it accumulates, so one accumulator carried
// across the whole reduction would be a chain of d_in / 4 rounded additions, several times the
// error of the reference's nn.lanes vector partial sums (src/core/nn.zig:68-126: 8 or 16 lanes of
// d_in / lanes products each, then a reduction). The reduction is therefore blocked: each chunk of
// c 16-wide units (16 c indices of the workgroup's range) runs as its own chain of 4 c
// instructions started at zero, and the chunk sums are added in order into the output's total.
// c ~ sqrt(d_in / 64) (proj_chunk) keeps the longest run of roundings near 4 sqrt(d_in / 16): 12
// steps at d_in 128, 28 at 768, 56 at 3072, in a fixed order that depends on d_in alone.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

// Tile shapes. SMALL: 64 tokens x 64 columns (one head), four waves = 2 (32 tokens) x 2 (column
// pairs 16 wq + {0, 32}). BIG: 128 tokens x 128 columns (two heads), eight waves = 4 (32 tokens) x
// 2 (heads), each wave all four 16-column blocks of its head.
constexpr int BM = 64;           // tokens per SMALL tile (and the unit of the split partials)
constexpr int BN = 64;           // columns per SMALL tile: one head
constexpr int GM = 8;            // token tiles that sweep the column tiles together
template <bool BIG> constexpr int tile_m() { return BIG ? 128 : 64; }
template <bool BIG> constexpr int tile_n() { return BIG ? 128 : 64; }
template <bool BIG> constexpr int threads() { return BIG ? 512 : 256; }
// Reduction step BK (16 or 32). LDS holds each tile of a step as 1 KB chunks, one per 16 rows x
// 16 reduction indices, in the order the matrix instructions read them (below): no padding, and
// every operand read is 64 lanes x 16 contiguous bytes.
template <int BK, bool BIG>
constexpr size_t proj_lds() { return (size_t)2 * (tile_m<BIG>() + tile_n<BIG>()) * BK * sizeof(float); }
static_assert(kSplitWorkspaceBytes == (size_t)1536 * BM * BN * sizeof(float), "split workspace size");
typedef __attribute__((address_space(3))) void* lds_void_ptr;
// 16 bytes per lane from global memory straight into LDS: lane l's go to lds + 16 l (lds the same
// for the whole wave).
__device__ __forceinline__ void load_lds16(const float* g, float* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void_ptr)lds, 16, 0, 0);
}

// Workgroup tile of a logical id: GM token tiles at a time go through all column tiles, token tile
// fastest, so the x rows of a group stay in L2 while the weight tiles stream past.
__device__ __forceinline__ void tile_of(int id, int m_tiles, int n_tiles, int& tm, int& tn) {
    const int per = GM * n_tiles;
    const int g = id / per, r = id - g * per;
    const int m0 = g * GM, gm = min(GM, m_tiles - m0);
    tm = m0 + r % gm;
    tn = r / gm;
}

// Element offset of token m (of p.tokens, p.seq per series row) in output sel.
__device__ __forceinline__ int64_t out_offset(const ProjParams& p, int sel, int m) {
    const int64_t tok = sel == 0 ? p.y0_tok : sel == 1 ? p.y1_tok : sel == 2 ? p.y2_tok : p.y3_tok;
    const int64_t bat = sel == 0 ? p.y0_batch : sel == 1 ? p.y1_batch : sel == 2 ? p.y2_batch : p.y3_batch;
    if (bat == 0) return (int64_t)m * tok;
    const int b = m / p.seq;
    return (int64_t)b * bat + (int64_t)(m - b * p.seq) * tok;
}

// The unary epilogues: nn.relu, and nn.silu (x / (1 + exp(-x))) of ResBlock(.silu).
__device__ __forceinline__ f32x4 epi_act(int epi, f32x4 v) {
    if (epi == kEpiRelu) return f32x4{fmaxf(v[0], 0.f), fmaxf(v[1], 0.f), fmaxf(v[2], 0.f), fmaxf(v[3], 0.f)};
    if (epi == kEpiSilu) {
#pragma clang fp contract(off)
        return f32x4{v[0] / (1.f + expf(-v[0])), v[1] / (1.f + expf(-v[1])), v[2] / (1.f + expf(-v[2])),
                     v[3] / (1.f + expf(-v[3]))};
    }
    return v;
}

// OUT: element type of the outputs, TSFM_DTYPE_* (0 f32, 1 bf16, 2 f16); the products and RoPE
// are f32 either way and the result is rounded once, to nearest even, when it is stored.
// The bf16x3 products: reduction indices per step of their kernels, and the bytes of one chunk of
// the pre-split operand layout (16 rows x 32 indices of one part, see split_planes).
constexpr int X3_BK = 32;
constexpr int kPlaneChunk = 1024;

// a = hi + mid + lo as bf16 pairs (two values per word, the first in the low half).
__device__ __forceinline__ void split3(f32x4 v, u32x2& hi, u32x2& mid, u32x2& lo) {
#pragma clang fp contract(off)
    auto widen = [](uint32_t w, int half) { return __uint_as_float(half ? (w & 0xffff0000u) : (w << 16)); };
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const float a = v[2 * i], b = v[2 * i + 1];
        const uint32_t h = pack2<true>(a, b);
        const float ra = a - widen(h, 0), rb = b - widen(h, 1);
        const uint32_t m = pack2<true>(ra, rb);
        const float sa = ra - widen(m, 0), sb = rb - widen(m, 1);
        hi[i] = h;
        mid[i] = m;
        lo[i] = pack2<true>(sa, sb);
    }
}

// The stores of a wave's finished sums (not split): sum[nb][mb] holds columns cq(nb) .. + 3 of the
// head at output column n0w (over all outputs) for token row0 + wm * 32 + mb * 16 + (lane & 15):
// alpha, RoPE of q and k, then bias and ReLU / SiLU / residual (f32) or the rounding (bf16, f16).
template <int OUT, bool BIG>
__device__ __forceinline__ void proj_store(const ProjParams& p, f32x4 (&sum)[BIG ? 4 : 2][2], int row0, int n0w, int wm,
                                           int wq, int lane) {
    constexpr int NB = BIG ? 4 : 2;
    const int sel = n0w / p.width, col = n0w - sel * p.width;
    const int c4 = 4 * (lane >> 4);
    auto cq = [&](int nb) { return (BIG ? 16 * nb : 16 * wq + 32 * nb) + c4; };  // column in the head
    void* const y = sel == 0 ? p.y0 : sel == 1 ? p.y1 : sel == 2 ? p.y2 : p.y3;
    const bool rope = p.rope_cos != nullptr && sel < 2;
#pragma unroll
    for (int mb = 0; mb < 2; mb++) {
        const int m = row0 + wm * 32 + mb * 16 + (lane & 15);
        if (m >= p.tokens) continue;
        if (p.alpha != 1.f) {  // gemmNT's alpha, applied to the finished sum (src/core/nn.zig:100)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) sum[nb][mb] *= p.alpha;
        }
        if (rope) {
            // Token t of series row b: row t of table (rope_row0 + b) / rope_rows_per_table; the
            // pairs (i, i + 32) are blocks (nb, nb + NB / 2).
            const int b = m / p.seq, tok = m - b * p.seq;
            const int table = p.rope_rows_per_table > 0 ? (p.rope_row0 + b) / p.rope_rows_per_table : 0;
#pragma unroll
            for (int k = 0; k < NB / 2; k++) {
                const int64_t at = (int64_t)table * p.rope_table_stride + (int64_t)tok * (kHeadDim / 2) + cq(k);
                rope4(sum[k][mb], sum[k + NB / 2][mb], ld4(p.rope_cos + at), ld4(p.rope_sin + at));
            }
        }
        const int64_t at = out_offset(p, sel, m) + col;
        if constexpr (OUT == 0) {
            float* const out = static_cast<float*>(y) + at;
            const float* const res = p.epi == kEpiResidual ? p.resid + (int64_t)m * p.resid_tok + col : nullptr;
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                if (col + cq(nb) >= p.width) continue;
                f32x4 v = sum[nb][mb];
                if (p.bias != nullptr) v = v + ld4(p.bias + col + cq(nb));  // nn.linear's bias (linearCols, nn.zig:254)
                if (p.epi == kEpiResidual) v = ld4(res + cq(nb)) + v;  // x + delta, one rounding
                else v = epi_act(p.epi, v);
                if (p.y_planes != nullptr) {
                    // Columns c .. c + 3 of row m in the pre-split layout of a (tokens x width)
                    // operand: chunk (m / 16, c / 32), lane 16 ((c % 32) / 8) + m % 16, bytes 2 (c % 8).
                    const int c = col + cq(nb), kcw = p.width / X3_BK;
                    u32x2 hp, mp, lp;
                    split3(v, hp, mp, lp);
                    uint8_t* const q = static_cast<uint8_t*>(p.y_planes) +
                                       ((int64_t)(m >> 4) * kcw + c / X3_BK) * 3 * kPlaneChunk +
                                       (16 * ((c % X3_BK) >> 3) + (m & 15)) * 16 + 2 * (c & 7);
                    *reinterpret_cast<u32x2*>(q) = hp;
                    *reinterpret_cast<u32x2*>(q + kPlaneChunk) = mp;
                    *reinterpret_cast<u32x2*>(q + 2 * kPlaneChunk) = lp;
                    continue;
                }
                st4(out + cq(nb), v);
            }
        } else {
            uint16_t* const out = static_cast<uint16_t*>(y) + at;
#pragma unroll
            for (int nb = 0; nb < NB; nb++) {
                const f32x4 v = sum[nb][mb];
                *reinterpret_cast<u32x2*>(out + cq(nb)) =
                    u32x2{pack2<OUT == 1>(v[0], v[1]), pack2<OUT == 1>(v[2], v[3])};
            }
        }
    }
}

// The partial sums of a split reduction: partial row m of split s holds all n_cols columns (every
// output side by side); proj_reduce adds the splits up in split order and finishes. Same wave
// layout as proj_store.
template <bool BIG>
__device__ __forceinline__ void proj_partial(const ProjParams& p, f32x4 (&sum)[BIG ? 4 : 2][2], int row0, int n0w,
                                             int wm, int wq, int lane, int split) {
    constexpr int NB = BIG ? 4 : 2;
    const int n_cols = p.width * p.n_out;
    const int col = n0w - (n0w / p.width) * p.width;
    const int c4 = 4 * (lane >> 4);
    auto cq = [&](int nb) { return (BIG ? 16 * nb : 16 * wq + 32 * nb) + c4; };  // column in the head
#pragma unroll
    for (int mb = 0; mb < 2; mb++) {
        const int m = row0 + wm * 32 + mb * 16 + (lane & 15);
        if (m >= p.tokens) continue;
        float* const out = p.partial + ((int64_t)split * p.tokens + m) * n_cols + n0w;
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
            if (col + cq(nb) < p.width) st4(out + cq(nb), sum[nb][mb]);
    }
}

template <int OUT, int BK, bool BIG>
__global__ __launch_bounds__(threads<BIG>()) __attribute__((amdgpu_waves_per_eu(4, 4))) void qkv_proj(ProjParams p) {
    constexpr int TM = tile_m<BIG>(), TN = tile_n<BIG>(), NT = threads<BIG>();
    constexpr int NB = BIG ? 4 : 2;                  // 16-column blocks per wave
    constexpr int NU = BK / 16;                      // 16-wide reduction units per step
    constexpr int CX = TM / 16 * NU, CW = TN / 16 * NU;  // 1 KB chunks of the x and weight tiles
    constexpr int NWAVE = NT / 64, PER = (CX + CW) / NWAVE;  // chunks a wave loads per step
    constexpr int STAGE = (TM + TN) * BK;            // floats per LDS stage
    static_assert(PER * NWAVE == CX + CW && CX % NWAVE == 0, "every wave loads PER chunks, all x or all weight");
    extern __shared__ __attribute__((aligned(16))) float smem[];  // [2][x chunks, weight chunks]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tm, tn;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int split = p.splits > 1 ? logical % p.splits : 0;  // this workgroup's share of the reduction
    tile_of(p.splits > 1 ? logical / p.splits : logical, p.m_tiles, p.n_tiles, tm, tn);
    const int n_cols = p.width * p.n_out;
    const int row0 = p.m_base + tm * TM;  // the tile's first token

    // Loader: wave w loads chunks w + NWAVE i (i < PER) of each step, HBM/L2 straight into LDS
    // (global_load_lds_dwordx4: lane l's 16 bytes land at the chunk's base + 16 l). Chunk e of the
    // x tile (of the weight tile: e - CX) is row block e / NU, unit e % NU; lane l loads row
    // (l & 15) of the block, reduction indices 16 (e % NU) + 4 (l >> 4) .. + 3 of the step. Rows
    // past the end are clamped to the last row: they feed only outputs that are not stored.
    const float* src[PER];
    int dst[PER];  // float offset of the chunk in a stage (the same for the whole wave)
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int ch = wave + NWAVE * i;
        const bool is_x = i < CX / NWAVE;
        const int e = is_x ? ch : ch - CX, r = (e / NU) * 16 + (lane & 15), kq = 16 * (e % NU) + 4 * (lane >> 4);
        if (is_x) {
            src[i] = p.x + (int64_t)min(row0 + r, p.tokens - 1) * p.x_tok + kq;
        } else {
            const int n = min(tn * TN + r, n_cols - 1);
            const int sel = n / p.width;
            const float* w = sel == 0 ? p.w0 : sel == 1 ? p.w1 : sel == 2 ? p.w2 : p.w3;
            src[i] = w + (int64_t)(n - sel * p.width) * p.w_ld + kq;
        }
        dst[i] = (is_x ? 0 : TM * BK) + e * 256;
    }
    auto stage_in = [&](int t, int buf) {
#pragma unroll
        for (int i = 0; i < PER; i++)
            load_lds16(src[i] + t * BK, smem + buf * STAGE + dst[i]);
    };

    // Wave layout: token block wm (32 tokens) and, SMALL, column pair wq (blocks wq and wq + 2 of
    // the head: a RoPE pair (i, i + 32) in one lane), BIG, head wq of the tile (blocks 0..3; pairs
    // (0, 2) and (1, 3)). colb(nb): the tile column of the wave's block nb.
    // Operand reads: lane l takes row (l & 15) of a 16-row block and the four reduction indices
    // 4 (l >> 4) .. + 3 of a 16-wide unit -- 16 bytes at 16 l in the block's chunk of the unit;
    // matrix instruction j uses element j, the same reduction index on both operands.
    const int wm = BIG ? (wave & 3) : (wave & 1), wq = BIG ? (wave >> 2) : (wave >> 1);
    auto colb = [&](int nb) { return BIG ? 64 * wq + 16 * nb : 16 * wq + 32 * nb; };
    const float* const xr = smem + (2 * wm * NU) * 256 + 4 * lane;
    const float* const wr = smem + TM * BK + 4 * lane;

    // tot: the output's total over the finished chunks; chk: the running chunk.
    // [column block nb][token block]: columns 4 (l >> 4) + r, token l & 15.
    f32x4 tot[NB][2], chk[NB][2];
#pragma unroll
    for (int a = 0; a < NB; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) tot[a][b] = chk[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int t0 = split * p.split_steps;
    const int steps = p.splits > 1 ? min(p.d_in / BK, t0 + p.split_steps) : p.d_in / BK;
    const int units = (steps - t0) * NU;  // 16-wide reduction units of this workgroup
    int cu = 0;                           // units done in the running chunk
    stage_in(t0, 0);
    __syncthreads();
    for (int t = t0; t < steps; t++) {
        const int buf = (t - t0) & 1;
        // The other stage was last read in step t - 1, which every wave has left (barrier below).
        if (t + 1 < steps) stage_in(t + 1, buf ^ 1);
#pragma unroll
        for (int c = 0; c < NU; c++) {
            const int u = (t - t0) * NU + c;
            f32x4 wa[NB], xb[2];
#pragma unroll
            for (int nb = 0; nb < NB; nb++) wa[nb] = ld4(wr + buf * STAGE + ((colb(nb) / 16) * NU + c) * 256);
#pragma unroll
            for (int mb = 0; mb < 2; mb++) xb[mb] = ld4(xr + buf * STAGE + (mb * NU + c) * 256);
            if (cu == 0) {  // a chunk starts: its chain begins at zero
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
#pragma unroll
                    for (int mb = 0; mb < 2; mb++)
                        chk[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[nb][0], xb[mb][0],
                                                                           f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            } else {
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
#pragma unroll
                    for (int mb = 0; mb < 2; mb++)
                        chk[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[nb][0], xb[mb][0], chk[nb][mb], 0, 0, 0);
            }
#pragma unroll
            for (int j = 1; j < 4; j++)
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
#pragma unroll
                    for (int mb = 0; mb < 2; mb++)
                        chk[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[nb][j], xb[mb][j], chk[nb][mb], 0, 0, 0);
            if (++cu == p.chunk || u == units - 1) {  // the chunk is done: into the total
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
#pragma unroll
                    for (int mb = 0; mb < 2; mb++) tot[nb][mb] += chk[nb][mb];
                cu = 0;
            }
        }
        __syncthreads();  // the loads of step t + 1 have landed; nobody reads stage buf any more
    }
    f32x4 (&sum)[NB][2] = tot;

    // Epilogue: the wave's columns of one output (or, with one output of a width that is not a
    // multiple of 64, columns of a partial head: groups of four columns past the width are not
    // stored). n0w: the output column (over all outputs) of the wave's head.
    const int n0w = tn * TN + (BIG ? 64 * wq : 0);
    if (n0w >= n_cols) return;
    if (p.splits > 1) {  // partial sums only; proj_reduce adds them up in split order and finishes
        proj_partial<BIG>(p, sum, row0, n0w, wm, wq, lane, split);
        return;
    }
    proj_store<OUT, BIG>(p, sum, row0, n0w, wm, wq, lane);
}

// ---- f32 products on the bf16 matrix cores --------------------------------------------------------
//
// The large products (128 x 128 tiles) can run their f32 arithmetic as bf16 products: each f32
// operand is split into three bf16 parts, a = a0 + a1 + a2 (a0 = bf16(a), a1 = bf16(a - a0),
// a2 = bf16(a - a0 - a1); both differences are exact in f32), so a0..a2 carry a's 24 significant
// bits. A product a b is the sum of the nine a_i b_j; each is exact in f32 (8 x 8 significant bits),
// and the three smallest (a1 b2, a2 b1, a2 b2: below 2^-24 of a b) are left out. The other six run
// on v_mfma_f32_16x16x32_bf16 into the f32 accumulator, smallest first (a2 b0, a0 b2, a1 b1, a1 b0,
// a0 b1, a0 b0). Each 16x16x32 instruction is 16 cycles against 32 for 16x16x4 f32 with an eighth
// of the work, so the six take 2.7x fewer matrix cycles than the f32 instructions, and the bf16
// matrix pipe runs beside the VALU (the f32 one does not). The accumulation stays blocked as in
// qkv_proj: chunks of 32-wide units, each its own chain started at zero, the chunk sums added in
// order.
//
// Staging: each step (32 reduction indices) the workgroup's 512 threads load the x and weight
// tiles (128 rows x 32 indices each) as 16-byte loads into registers one step ahead, split them,
// and write the three bf16 planes into the other LDS stage in the matrix instruction's operand
// order: per 16 rows x 32 indices, lane l's 16 bytes (row l & 15, indices 8 (l >> 4) .. + 7) at 16 l.
// 48 KB per stage, two stages: one workgroup (8 waves) per CU.
// Per tile shape: the bytes of one bf16 plane of one tile (rows x 32 indices x 2 bytes), the three
// planes of a tile, a stage (weight tile, then x tile), and both stages.
template <bool BIG> constexpr int x3_plane() { return tile_m<BIG>() * X3_BK * 2; }
template <bool BIG> constexpr int x3_stage() { return 2 * 3 * x3_plane<BIG>(); }
template <bool BIG> constexpr size_t x3_lds() { return 2 * (size_t)x3_stage<BIG>(); }
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) u32x4* lds_u32x4_p;
typedef __attribute__((address_space(3))) u32x2* lds_u32x2_p;

__device__ __forceinline__ f32x4 mfma_x3(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b), c, 0,
                                                   0, 0);
}

// Tiles and waves as qkv_proj's: BIG 128 x 128 (8 waves of 32 tokens x one head, each its four
// column blocks), SMALL 64 x 64 (4 waves of 32 tokens x column blocks wq and wq + 2). Per output
// element the products and their order depend on d_in and the chunk alone, so both shapes give the
// same bits for the same row.
template <int OUT, bool BIG>
__global__ __launch_bounds__(threads<BIG>()) __attribute__((amdgpu_waves_per_eu(BIG ? 2 : 3, BIG ? 2 : 3))) void
qkv_proj_x3(ProjParams p) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int T = tile_m<BIG>(), NT = threads<BIG>(), NB = BIG ? 4 : 2;
    constexpr int PLANE = x3_plane<BIG>(), TILE = 3 * PLANE, STAGE = x3_stage<BIG>();
    static_assert(T * 8 == 2 * NT, "each thread loads two 16-byte slots of each tile per step");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tm, tn;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int split = p.splits > 1 ? logical % p.splits : 0;  // this workgroup's share of the reduction
    tile_of(p.splits > 1 ? logical / p.splits : logical, p.m_tiles, p.n_tiles, tm, tn);
    const int n_cols = p.width * p.n_out;
    const int row0 = p.m_base + tm * T;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)smem;

    // Loader: 16-byte slot e = tid + NT i (i < 2) of each tile, taken in plane order so a wave's
    // LDS writes cover 512 contiguous bytes (no bank conflicts): 16-row block e / 128; within it,
    // lane-slot s = (e % 128) / 2 holds row s % 16, indices 8 (s / 16) .. + 7, of which the slot
    // takes the half e % 2: indices 8 (s / 16) + 4 (e % 2) .. + 3 of the step. Rows past the end
    // are clamped to the last row (they feed only outputs that are not stored). dst: the slot's
    // byte offset in a plane (16-row block, then lane (row, index / 8)).
    const float* wsrc[2];
    const float* xsrc[2];
    uint32_t dst[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int e = tid + NT * i, sl = (e & 127) >> 1;
        const int r = 16 * (e >> 7) + (sl & 15), kq = 8 * (sl >> 4) + 4 * (e & 1);
        const int n = min(tn * T + r, n_cols - 1), sel = n / p.width;
        const float* w = sel == 0 ? p.w0 : sel == 1 ? p.w1 : sel == 2 ? p.w2 : p.w3;
        wsrc[i] = w + (int64_t)(n - sel * p.width) * p.w_ld + kq;
        xsrc[i] = p.x + (int64_t)min(row0 + r, p.tokens - 1) * p.x_tok + kq;
        dst[i] = (uint32_t)((r >> 4) * 1024 + ((kq >> 3) * 16 + (r & 15)) * 16 + (kq & 7) * 2);
    }
    f32x4 pw[2], px[2];
    auto load = [&](int t) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            pw[i] = ld4(wsrc[i] + t * X3_BK);
            px[i] = ld4(xsrc[i] + t * X3_BK);
        }
    };
    auto store = [&](int buf) {
        const uint32_t st = lds0 + (uint32_t)buf * STAGE;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            u32x2 h, m, l;
            split3(pw[i], h, m, l);
            *(lds_u32x2_p)(uintptr_t)(st + dst[i]) = h;
            *(lds_u32x2_p)(uintptr_t)(st + PLANE + dst[i]) = m;
            *(lds_u32x2_p)(uintptr_t)(st + 2 * PLANE + dst[i]) = l;
            split3(px[i], h, m, l);
            *(lds_u32x2_p)(uintptr_t)(st + TILE + dst[i]) = h;
            *(lds_u32x2_p)(uintptr_t)(st + TILE + PLANE + dst[i]) = m;
            *(lds_u32x2_p)(uintptr_t)(st + TILE + 2 * PLANE + dst[i]) = l;
        }
    };

    // Wave (wm, wq): tokens 32 wm .. + 31 (blocks 2 wm, 2 wm + 1); column block cb(nb).
    const int wm = BIG ? (wave & 3) : (wave & 1), wq = BIG ? (wave >> 2) : (wave >> 1);
    auto cb = [&](int nb) { return BIG ? 4 * wq + nb : wq + 2 * nb; };
    f32x4 tot[NB][2], chk[NB][2];
#pragma unroll
    for (int a = 0; a < NB; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) tot[a][b] = chk[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Steps [t0, steps) of 32 indices: the whole reduction, or this split's share (split_steps
    // counts 16-wide units and is even when the reduction is split for this kernel).
    const int t0 = p.splits > 1 ? split * (p.split_steps / 2) : 0;
    const int steps = p.splits > 1 ? min(p.d_in / X3_BK, t0 + p.split_steps / 2) : p.d_in / X3_BK;
    int cu = 0;  // units done in the running chunk
    load(t0);
    store(0);
    __syncthreads();
    for (int t = t0; t < steps; t++) {
        const uint32_t st = lds0 + (uint32_t)((t - t0) & 1) * STAGE;
        if (t + 1 < steps) load(t + 1);
        u32x4 a[3][NB], b[3][2];
#pragma unroll
        for (int pl = 0; pl < 3; pl++) {
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                a[pl][nb] = *(lds_u32x4_p)(uintptr_t)(st + pl * PLANE + cb(nb) * 1024 + lane * 16);
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
                b[pl][mb] = *(lds_u32x4_p)(uintptr_t)(st + TILE + pl * PLANE + (2 * wm + mb) * 1024 + lane * 16);
        }
        // The six products, smallest first: (weight part, x part).
        constexpr int kA[6] = {2, 0, 1, 1, 0, 0}, kB[6] = {0, 2, 1, 0, 1, 0};
        const bool fresh = cu == 0;  // a chunk starts: its chain begins at zero
#pragma unroll
        for (int j = 0; j < 6; j++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
#pragma unroll
                for (int mb = 0; mb < 2; mb++)
                    chk[nb][mb] = mfma_x3(a[kA[j]][nb], b[kB[j]][mb],
                                          (j == 0 && fresh) ? f32x4{0.f, 0.f, 0.f, 0.f} : chk[nb][mb]);
        if (++cu == p.chunk || t == steps - 1) {
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
#pragma unroll
                for (int mb = 0; mb < 2; mb++) tot[nb][mb] += chk[nb][mb];
            cu = 0;
        }
        // Stage t + 1 goes to the other buffer, last read in step t - 1 (every wave has passed the
        // barrier after it).
        if (t + 1 < steps) store((t + 1 - t0) & 1);
        __syncthreads();
    }
    const int n0w = tn * T + (BIG ? 64 * wq : 0);
    if (n0w >= n_cols) return;
    if (p.splits > 1) {
        proj_partial<BIG>(p, tot, row0, n0w, wm, wq, lane, split);
        return;
    }
    proj_store<OUT, BIG>(p, tot, row0, n0w, wm, wq, lane);
}

// ---- pre-split operands -----------------------------------------------------------------------
//
// When the calling entry point provides a workspace (PlaneWorkspace), x and the weights are split
// once per product by split_planes into the layout the matrix instruction reads, and qkv_proj_x3p
// takes its tiles from there straight into LDS (buffer_load ... lds): no staging registers and no
// VALU split inside the product, three LDS stages (DMA two steps ahead), one barrier per step.
// Same split, same products in the same order as qkv_proj_x3, so the two give the same bits.
//
// Layout of a pre-split (rows x d_in) matrix, KC = d_in / 32: 1 KB chunks, one per (16-row block rb,
// 32-index step kc, part pl), at ((rb KC + kc) 3 + pl) KB; in a chunk, lane l's 16 bytes (row
// 16 rb + (l & 15), indices 32 kc + 8 (l >> 4) .. + 7, as bf16) at 16 l. Rows past the matrix are
// zeros.
struct SplitSrc {
    const float* src[4];  // row r comes from src[r / per], row r % per
    int64_t ld;
    int32_t per, rows, kc;
};
__global__ __launch_bounds__(256) void split_planes(SplitSrc s, uint8_t* __restrict__ dst) {
    const int64_t c = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // chunk (rb, kc)
    const int lane = threadIdx.x & 63;
    if (c >= (int64_t)((s.rows + 15) / 16) * s.kc) return;
    const int rb = (int)(c / s.kc), kc = (int)(c - (int64_t)rb * s.kc);
    const int row = rb * 16 + (lane & 15), k0 = kc * 32 + 8 * (lane >> 4);
    f32x4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
    if (row < s.rows) {
        const int sel = row / s.per;
        const float* r = s.src[sel] + (int64_t)(row - sel * s.per) * s.ld + k0;
        a = ld4(r);
        b = ld4(r + 4);
    }
    u32x2 h0, m0, l0, h1, m1, l1;
    split3(a, h0, m0, l0);
    split3(b, h1, m1, l1);
    uint8_t* const out = dst + c * 3 * kPlaneChunk + 16 * lane;
    *reinterpret_cast<u32x4*>(out) = u32x4{h0[0], h0[1], h1[0], h1[1]};
    *reinterpret_cast<u32x4*>(out + kPlaneChunk) = u32x4{m0[0], m0[1], m1[0], m1[1]};
    *reinterpret_cast<u32x4*>(out + 2 * kPlaneChunk) = u32x4{l0[0], l0[1], l1[0], l1[1]};
}

// rmsNorm of 16 rows per workgroup into the pre-split layout: each wave reduces four rows with the
// lane mapping of rms_norm_rows (so the norms are the same bits), then the workgroup writes the
// rows' chunks, 1 KB per wave at a time.
__global__ __launch_bounds__(256) void rms_norm_planes(const float* __restrict__ x, int64_t x_tok,
                                                       uint8_t* __restrict__ dst, const float* __restrict__ scale,
                                                       int rows, int dim, float eps) {
    __shared__ float inv_s[16];
    const int rb = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 4 * wave + i, row = rb * 16 + r;
        if (row >= rows) continue;  // wave-uniform
        const float* xr = x + (int64_t)row * x_tok;
        float ss = 0.f;
        for (int c = 4 * lane; c < dim; c += 256) ss = sumsq4(ss, ld4(xr + c));
        const float inv = rms_inv(ss, dim, eps);
        if (lane == 0) inv_s[r] = inv;
    }
    __syncthreads();
    const int kc = dim / X3_BK, r = lane & 15, row = rb * 16 + r;
    for (int k = wave; k < kc; k += 4) {
        const int c0 = k * X3_BK + 8 * (lane >> 4);
        f32x4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
        if (row < rows) {
            const float* xr = x + (int64_t)row * x_tok + c0;
            a = rms_apply(ld4(xr), inv_s[r], ld4(scale + c0));
            b = rms_apply(ld4(xr + 4), inv_s[r], ld4(scale + c0 + 4));
        }
        u32x2 h0, m0, l0, h1, m1, l1;
        split3(a, h0, m0, l0);
        split3(b, h1, m1, l1);
        uint8_t* const out = dst + ((int64_t)rb * kc + k) * 3 * kPlaneChunk + 16 * lane;
        *reinterpret_cast<u32x4*>(out) = u32x4{h0[0], h0[1], h1[0], h1[1]};
        *reinterpret_cast<u32x4*>(out + kPlaneChunk) = u32x4{m0[0], m0[1], m1[0], m1[1]};
        *reinterpret_cast<u32x4*>(out + 2 * kPlaneChunk) = u32x4{l0[0], l0[1], l1[0], l1[1]};
    }
}

template <int OUT, bool BIG>
__global__ __launch_bounds__(threads<BIG>()) __attribute__((amdgpu_waves_per_eu(2, 2))) void qkv_proj_x3p(ProjParams p) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int T = tile_m<BIG>(), NT = threads<BIG>(), NB = BIG ? 4 : 2;
    constexpr int PLANE = x3_plane<BIG>(), TILE = 3 * PLANE, STAGE = x3_stage<BIG>();
    constexpr int RB = T / 16, NWAVE = NT / 64, PER = 6 * RB / NWAVE;  // chunks a wave loads per step
    static_assert(PER * NWAVE == 6 * RB && PER == 6, "six 1 KB chunks per wave and step");
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tm, tn;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int split = p.splits > 1 ? logical % p.splits : 0;  // this workgroup's share of the reduction
    tile_of(p.splits > 1 ? logical / p.splits : logical, p.m_tiles, p.n_tiles, tm, tn);
    const int n_cols = p.width * p.n_out;
    const int row0 = p.m_base + tm * T;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)smem;

    // The tile's row blocks of the pre-split weights (columns) and x (tokens), through descriptors
    // that end with the matrix: blocks past it read as zeros (they feed only outputs not stored).
    const int kc = p.d_in / X3_BK;
    const int rbw = tn * RB, rbx = row0 / 16;
    const int nw = max(0, min(RB, (n_cols + 15) / 16 - rbw)), nx = max(0, min(RB, (p.tokens + 15) / 16 - rbx));
    const u32x4 wd = buf_desc(static_cast<const uint8_t*>(p.wp) + (int64_t)rbw * kc * 3 * kPlaneChunk,
                              (uint32_t)((int64_t)nw * kc * 3 * kPlaneChunk));
    const u32x4 xd = buf_desc(static_cast<const uint8_t*>(p.xp) + (int64_t)rbx * kc * 3 * kPlaneChunk,
                              (uint32_t)((int64_t)nx * kc * 3 * kPlaneChunk));
    // Step t into stage buf: chunk c = wave + NWAVE i of the step is (weights, then x) part pl of row
    // block rb, landing where qkv_proj_x3 writes it.
    auto issue = [&](int t, int buf) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = wave + NWAVE * i, side = c / (3 * RB), rem = c - side * 3 * RB;
            const int pl = rem / RB, rb = rem - pl * RB;
            const uint32_t src = (uint32_t)(((rb * kc + t) * 3 + pl) * kPlaneChunk) + 16u * lane;
            dma16(side ? xd : wd, lds0 + (uint32_t)(buf * STAGE + side * TILE + pl * PLANE + rb * kPlaneChunk), src,
                  0u);
        }
    };

    const int wm = BIG ? (wave & 3) : (wave & 1), wq = BIG ? (wave >> 2) : (wave >> 1);
    auto cb = [&](int nb) { return BIG ? 4 * wq + nb : wq + 2 * nb; };
    f32x4 tot[NB][2], chk[NB][2];
#pragma unroll
    for (int a = 0; a < NB; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) tot[a][b] = chk[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int t0 = p.splits > 1 ? split * (p.split_steps / 2) : 0;
    const int steps = p.splits > 1 ? min(kc, t0 + p.split_steps / 2) : kc;
    int cu = 0;  // units done in the running chunk
    issue(t0, 0);
    if (t0 + 1 < steps) issue(t0 + 1, 1);
    for (int t = t0; t < steps; t++) {
        // This wave's chunks of step t have landed (those of step t + 1 may still be in flight),
        // then every wave's; every wave has also left step t - 1, whose stage step t + 2 reuses.
        if (t + 1 < steps) asm volatile("s_waitcnt vmcnt(6)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (t + 2 < steps) issue(t + 2, (t + 2 - t0) % 3);
        const uint32_t st = lds0 + (uint32_t)((t - t0) % 3) * STAGE;
        u32x4 a[3][NB], b[3][2];
#pragma unroll
        for (int pl = 0; pl < 3; pl++) {
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
                a[pl][nb] = *(lds_u32x4_p)(uintptr_t)(st + pl * PLANE + cb(nb) * 1024 + lane * 16);
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
                b[pl][mb] = *(lds_u32x4_p)(uintptr_t)(st + TILE + pl * PLANE + (2 * wm + mb) * 1024 + lane * 16);
        }
        constexpr int kA[6] = {2, 0, 1, 1, 0, 0}, kB[6] = {0, 2, 1, 0, 1, 0};
#pragma unroll
        for (int j = 0; j < 6; j++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
#pragma unroll
                for (int mb = 0; mb < 2; mb++) chk[nb][mb] = mfma_x3(a[kA[j]][nb], b[kB[j]][mb], chk[nb][mb]);
        if (++cu == p.chunk || t == steps - 1) {  // the chunk is done: into the total, the next starts at zero
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
#pragma unroll
                for (int mb = 0; mb < 2; mb++) {
                    tot[nb][mb] += chk[nb][mb];
                    chk[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
            cu = 0;
        }
    }
    const int n0w = tn * T + (BIG ? 64 * wq : 0);
    if (n0w >= n_cols) return;
    if (p.splits > 1) {
        proj_partial<BIG>(p, tot, row0, n0w, wm, wq, lane, split);
        return;
    }
    proj_store<OUT, BIG>(p, tot, row0, n0w, wm, wq, lane);
}
template <bool BIG> constexpr size_t x3p_lds() { return 3 * (size_t)x3_stage<BIG>(); }  // three stages

// The widest tiles, for the largest pre-split products: 256 tokens x 128 columns per workgroup,
// eight waves of 64 tokens x one 64-column head each (4 x 4 blocks of 16 x 16): per 32-index step
// a wave reads 24 KB of operands for 96 matrix instructions, against 18 KB for 48 with 32-token
// waves. Two LDS stages of 72 KB (DMA one step ahead). Same products, same order, same bits.
constexpr int kWideM = 256;
constexpr int kWideStage = 3 * (kWideM + 128) * X3_BK * 2;  // bytes: weights then x, three parts each
template <int OUT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void qkv_proj_x3w(ProjParams p) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int RBW = 128 / 16, RBX = kWideM / 16, NCH = 3 * (RBW + RBX), PER = NCH / 8;
    constexpr int PW = RBW * 1024, PX = RBX * 1024, XOFF = 3 * PW;  // part sizes, x offset (bytes)
    static_assert(PER * 8 == NCH, "every wave loads PER chunks");
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tm, tn;
    tile_of(xcd_remap(blockIdx.x, gridDim.x), p.m_tiles, p.n_tiles, tm, tn);
    const int n_cols = p.width * p.n_out;
    const int row0 = p.m_base + tm * kWideM;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)smem;
    const int kc = p.d_in / X3_BK;
    const int rbw = tn * RBW, rbx = row0 / 16;
    const int nw = max(0, min(RBW, (n_cols + 15) / 16 - rbw)), nx = max(0, min(RBX, (p.tokens + 15) / 16 - rbx));
    const u32x4 wd = buf_desc(static_cast<const uint8_t*>(p.wp) + (int64_t)rbw * kc * 3 * kPlaneChunk,
                              (uint32_t)((int64_t)nw * kc * 3 * kPlaneChunk));
    const u32x4 xd = buf_desc(static_cast<const uint8_t*>(p.xp) + (int64_t)rbx * kc * 3 * kPlaneChunk,
                              (uint32_t)((int64_t)nx * kc * 3 * kPlaneChunk));
    // Step t into stage buf: chunk c = wave + 8 i is weight part c / RBW, block c % RBW (c < 3 RBW),
    // else x part, block of c - 3 RBW.
    auto issue = [&](int t, int buf) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int c = wave + 8 * i;
            const bool is_x = c >= 3 * RBW;
            const int e = is_x ? c - 3 * RBW : c, per = is_x ? RBX : RBW;
            const int pl = e / per, rb = e - pl * per;
            const uint32_t src = (uint32_t)(((rb * kc + t) * 3 + pl) * kPlaneChunk) + 16u * lane;
            const uint32_t dst = (uint32_t)(buf * kWideStage + (is_x ? XOFF + pl * PX : pl * PW) + rb * kPlaneChunk);
            dma16(is_x ? xd : wd, lds0 + dst, src, 0u);
        }
    };

    const int wm = wave & 3, wq = wave >> 2;  // tokens 64 wm .. + 63, head wq of the tile
    f32x4 tot[4][4], chk[4][4];  // [column block nb][token block mb]
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) tot[a][b] = chk[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    int cu = 0;  // units done in the running chunk
    issue(0, 0);
    for (int t = 0; t < kc; t++) {
        // This step's chunks have landed, for this wave and then every wave; every wave has left
        // step t - 1, whose stage step t + 1 reuses.
        asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (t + 1 < kc) issue(t + 1, (t + 1) & 1);
        const uint32_t st = lds0 + (uint32_t)(t & 1) * kWideStage;
        u32x4 a[3][4], b[3][4];
#pragma unroll
        for (int pl = 0; pl < 3; pl++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                a[pl][k] = *(lds_u32x4_p)(uintptr_t)(st + pl * PW + (4 * wq + k) * 1024 + lane * 16);
                b[pl][k] = *(lds_u32x4_p)(uintptr_t)(st + XOFF + pl * PX + (4 * wm + k) * 1024 + lane * 16);
            }
        constexpr int kA[6] = {2, 0, 1, 1, 0, 0}, kB[6] = {0, 2, 1, 0, 1, 0};
#pragma unroll
        for (int j = 0; j < 6; j++)
#pragma unroll
            for (int nb = 0; nb < 4; nb++)
#pragma unroll
                for (int mb = 0; mb < 4; mb++) chk[nb][mb] = mfma_x3(a[kA[j]][nb], b[kB[j]][mb], chk[nb][mb]);
        if (++cu == p.chunk || t == kc - 1) {  // the chunk is done: into the total, the next starts at zero
#pragma unroll
            for (int nb = 0; nb < 4; nb++)
#pragma unroll
                for (int mb = 0; mb < 4; mb++) {
                    tot[nb][mb] += chk[nb][mb];
                    chk[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
            cu = 0;
        }
    }
    const int n0w = tn * 128 + 64 * wq;
    if (n0w >= n_cols) return;
    // Token blocks (0, 1) and (2, 3) are the 32-token rows 2 wm and 2 wm + 1 of proj_store's layout.
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++) {
        f32x4 s2[4][2];
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
            s2[nb][0] = tot[nb][2 * h2];
            s2[nb][1] = tot[nb][2 * h2 + 1];
        }
        proj_store<OUT, true>(p, s2, row0, n0w, 2 * wm + h2, wq, lane);
    }
}

// The epilogue of four summed columns c .. c + 3 (of all n_out outputs side by side) of token m:
// alpha, and with one output bias, ReLU or residual; f32 store into the output the columns
// belong to (width is a multiple of 4, so a group never straddles two outputs).
__device__ __forceinline__ void finish4(const ProjParams& p, int m, int c, f32x4 v) {
    if (p.alpha != 1.f) v *= p.alpha;
    const int sel = c / p.width, col = c - sel * p.width;
    if (p.bias != nullptr) v = v + ld4(p.bias + col);
    if (p.epi == kEpiResidual) v = ld4(p.resid + (int64_t)m * p.resid_tok + col) + v;
    else v = epi_act(p.epi, v);
    float* const y = static_cast<float*>(sel == 0 ? p.y0 : sel == 1 ? p.y1 : sel == 2 ? p.y2 : p.y3);
    st4(y + out_offset(p, sel, m) + col, v);
}

// The split partials of four columns (split s at at + s stride), summed in split order; the loads
// of four splits at a time are issued before their adds.
__device__ __forceinline__ f32x4 split_sum(const float* at, int64_t stride, int splits) {
    f32x4 v = ld4(at);
    for (int s = 1; s < splits; s += 4) {
        f32x4 t[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (s + j < splits) t[j] = ld4(at + (s + j) * stride);
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (s + j < splits) v = v + t[j];
    }
    return v;
}

// Sum of the split partials in split order (deterministic), then the epilogue: alpha, and with one
// output bias, ReLU or residual; f32 store into the output the column belongs to. One thread per
// four columns of a token (width is a multiple of 4, so a group never straddles two outputs).
__global__ __launch_bounds__(256) void proj_reduce(ProjParams p) {
    const int n_cols = p.width * p.n_out, q = n_cols / 4;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.tokens * q) return;
    const int m = (int)(idx / q), c = (int)(idx % q) * 4;
    finish4(p, m, c, split_sum(p.partial + (int64_t)m * n_cols + c, (int64_t)p.tokens * n_cols, p.splits));
}

// proj_reduce for one output followed by the row norm of the finished rows: one wave per token
// row sums the partials of its four-column groups in split order, applies the epilogue, stores
// y0, and keeps the row's sum of squares; then norm_out = y0 * inv * norm_scale. The row norm's
// grouping and order are rms_norm_rows', so the result has the same bits as the two launches.
// Rows up to 256 KEEP wide stay in registers between the two passes.
__global__ __launch_bounds__(256) void proj_reduce_norm(ProjParams p) {
    constexpr int KEEP = 4;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= p.tokens) return;
    const int W = p.width;
    float* const y = static_cast<float*>(p.y0) + out_offset(p, 0, row);
    const int64_t stride = (int64_t)p.tokens * W;
    auto finish = [&](int c) {
        f32x4 v = split_sum(p.partial + (int64_t)row * W + c, stride, p.splits);
        if (p.alpha != 1.f) v *= p.alpha;
        if (p.bias != nullptr) v = v + ld4(p.bias + c);
        if (p.epi == kEpiResidual) v = ld4(p.resid + (int64_t)row * p.resid_tok + c) + v;
        else v = epi_act(p.epi, v);
        st4(y + c, v);
        return v;
    };
    float ss = 0.f;
    float* const o = p.norm_out + (int64_t)row * p.norm_out_tok;
    if (W <= 256 * KEEP) {
        f32x4 keep[KEEP];
#pragma unroll
        for (int i = 0; i < KEEP; i++) {
            const int c = 4 * lane + 256 * i;
            if (c < W) {
                keep[i] = finish(c);
                ss = sumsq4(ss, keep[i]);
            }
        }
        const float inv = rms_inv(ss, W, p.norm_eps);
#pragma unroll
        for (int i = 0; i < KEEP; i++) {
            const int c = 4 * lane + 256 * i;
            if (c < W) st4(o + c, rms_apply(keep[i], inv, ld4(p.norm_scale + c)));
        }
        return;
    }
    for (int c = 4 * lane; c < W; c += 256) ss = sumsq4(ss, finish(c));
    const float inv = rms_inv(ss, W, p.norm_eps);
    for (int c = 4 * lane; c < W; c += 256) st4(o + c, rms_apply(ld4(y + c), inv, ld4(p.norm_scale + c)));
}

// Products of at most 16 tokens (the Chronos-Bolt decoder: one token per series), f32 outputs, no
// RoPE. Such a product is a few MB of weights read once: it is bound by how many loads are in
// flight, not by the matrix cores. A workgroup takes one 16-column tile of every token and its
// sixteen waves split the reduction: wave w takes the 16-wide units [w U / 16, (w + 1) U / 16) of
// U = d_in / 16 and issues the loads of up to SKB of them at once, straight from HBM/L2 into
// registers in the matrix instruction's layout (lane l: row l & 15 of a 16-row block, indices
// 4 (l >> 4) .. + 3 of the unit), then multiplies them, accumulating blockwise as qkv_proj does.
// The sixteen 16 x 16 partials meet in LDS and are added in wave order, then the epilogue: one
// launch where a split over workgroups would need a second one for the sums.
constexpr int SKW = 16;  // waves of a workgroup
constexpr int SKB = 8;   // units a wave has in flight
constexpr int kSkinnyTokens = 16;
// Longer reductions read more weight bytes per column tile than the few CUs of a 16-token launch
// (one per 64 columns) pull in time; they split over workgroups instead (measured at d_in 2048:
// 13 us in one launch, 7 + 4 us split and summed).
constexpr int kSkinnyMaxIn = 1024;
constexpr size_t kSkinnyLds = (size_t)SKW * kSkinnyTokens * 16 * sizeof(float);
__global__ __launch_bounds__(64 * SKW) void proj_skinny(ProjParams p) {
    extern __shared__ __attribute__((aligned(16))) float smem[];  // [wave][token][16 columns]
    __shared__ float inv_s[kSkinnyTokens];
    static_assert(SKW == kSkinnyTokens, "one wave per token row for the input norm");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n_cols = p.width * p.n_out, tn = blockIdx.x;
    const int units = p.d_in / 16;
    const int u0 = wave * units / SKW, u1 = (wave + 1) * units / SKW;
    const int r = lane & 15, kq = 4 * (lane >> 4);
    const float* const xr = p.x + (int64_t)min(r, p.tokens - 1) * p.x_tok + kq;
    const bool in_norm = p.in_norm_scale != nullptr;  // uniform
    if (in_norm) {
        // Wave w: the norm of token row w (clamped as the loads are), with rms_norm_rows' lane
        // mapping and order, so the normalised inputs have its bits.
        const float* const xw = p.x + (int64_t)min(wave, p.tokens - 1) * p.x_tok;
        float ss = 0.f;
        for (int i = 4 * lane; i < p.d_in; i += 256) ss = sumsq4(ss, ld4(xw + i));
        const float inv = rms_inv(ss, p.d_in, p.in_norm_eps);
        if (lane == 0) inv_s[wave] = inv;
        __syncthreads();
    }
    const float inv_r = in_norm ? inv_s[r] : 1.f;
    const float* const sr = in_norm ? p.in_norm_scale + kq : nullptr;
    const float* wr;
    {  // weight row of the lane's column (clamped past the last column)
        const int n = min(tn * 16 + r, n_cols - 1);
        const int sel = n / p.width;
        const float* w = sel == 0 ? p.w0 : sel == 1 ? p.w1 : sel == 2 ? p.w2 : p.w3;
        wr = w + (int64_t)(n - sel * p.width) * p.w_ld + kq;
    }
    f32x4 tot = {0.f, 0.f, 0.f, 0.f}, chk = tot;
    int cu = 0;  // units done in the running chunk
    for (int b0 = u0; b0 < u1; b0 += SKB) {
        const int nb = min(SKB, u1 - b0);
        f32x4 xs[SKB], ws[SKB];
#pragma unroll
        for (int i = 0; i < SKB; i++) {
            if (i < nb) {
                xs[i] = ld4(xr + 16 * (b0 + i));
                ws[i] = ld4(wr + 16 * (b0 + i));
            }
        }
        if (in_norm) {
#pragma unroll
            for (int i = 0; i < SKB; i++)
                if (i < nb) xs[i] = rms_apply(xs[i], inv_r, ld4(sr + 16 * (b0 + i)));
        }
#pragma unroll
        for (int i = 0; i < SKB; i++) {
            if (i >= nb) break;
            chk = __builtin_amdgcn_mfma_f32_16x16x4f32(ws[i][0], xs[i][0], cu == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : chk,
                                                       0, 0, 0);
#pragma unroll
            for (int j = 1; j < 4; j++) chk = __builtin_amdgcn_mfma_f32_16x16x4f32(ws[i][j], xs[i][j], chk, 0, 0, 0);
            if (++cu == p.chunk || b0 + i == u1 - 1) {
                tot += chk;
                cu = 0;
            }
        }
    }
    // Lane l holds columns 4 (l >> 4) .. + 3 of token l & 15.
    st4(smem + (wave * kSkinnyTokens + r) * 16 + kq, tot);
    __syncthreads();
    if (tid >= kSkinnyTokens * 4) return;
    const int m = tid >> 2, c4 = 4 * (tid & 3), c = tn * 16 + c4;
    if (m >= p.tokens || c >= n_cols) return;
    f32x4 v = ld4(smem + m * 16 + c4);
    for (int w = 1; w < SKW; w++) v = v + ld4(smem + (w * kSkinnyTokens + m) * 16 + c4);
    finish4(p, m, c, v);
}

}  // namespace

namespace {

// The split-partials buffer of the calling thread's current library call (SplitWorkspace).
thread_local float* t_split_ws = nullptr;
// The pre-split operand buffer of the calling thread's current library call (PlaneWorkspace).
thread_local void* t_plane_ws = nullptr;
thread_local size_t t_plane_bytes = 0;

}  // namespace

SplitWorkspace::SplitWorkspace(float* buf) : prev_(t_split_ws) { t_split_ws = buf; }
SplitWorkspace::~SplitWorkspace() { t_split_ws = prev_; }
PlaneWorkspace::PlaneWorkspace(void* buf, size_t bytes) : prev_(t_plane_ws), prev_bytes_(t_plane_bytes) {
    t_plane_ws = buf;
    t_plane_bytes = buf != nullptr ? bytes : 0;
}
PlaneWorkspace::~PlaneWorkspace() {
    t_plane_ws = prev_;
    t_plane_bytes = prev_bytes_;
}
size_t proj_plane_bytes(int64_t tokens, int64_t d_in, int64_t n_cols) {
    if (tokens <= 0 || d_in <= 0 || n_cols <= 0 || d_in % X3_BK) return 0;
    return (size_t)((tokens + 15) / 16 + (n_cols + 15) / 16) * (size_t)(d_in / X3_BK) * 3 * kPlaneChunk;
}
size_t plane_operand_bytes(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0 || cols % X3_BK) return 0;
    return (size_t)((rows + 15) / 16) * (size_t)(cols / X3_BK) * 3 * kPlaneChunk;
}
// Products of at least 2^30 multiply-adds run on pre-split operands when a workspace is lent: the
// split launches cost more than they save on smaller ones.
static bool planes_pay(int64_t tokens, int64_t d_in, int64_t n_cols) {
    return d_in % X3_BK == 0 && tokens * n_cols * d_in >= ((int64_t)1 << 30);
}
bool proj_planes_ready(int64_t tokens, int64_t d_in, int64_t n_cols) {
    return t_plane_ws != nullptr && planes_pay(tokens, d_in, n_cols) &&
           plane_operand_bytes(n_cols, d_in) <= t_plane_bytes;
}
hipError_t launch_rms_norm_planes(const float* x, int64_t x_tok, void* planes, const float* scale, int rows, int dim,
                                  float eps, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (dim <= 0 || dim % X3_BK) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rms_norm_planes, dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, stream, x, x_tok,
                       static_cast<uint8_t*>(planes), scale, rows, dim, eps);
    return hipGetLastError();
}

namespace {

// The unsplit product. BIG tiles when there are enough of them for every CU; SMALL ones take
// 32-wide steps when d_in allows (half the step barriers), else 16-wide. The accumulation chunks
// are the same units of 16 p.chunk indices either way, so the result depends on neither the step
// width nor the tile shape, and one product may mix the two.
constexpr int64_t kBigTilesMin = 256;
template <int OUT>
hipError_t launch_small(ProjParams p, hipStream_t stream) {
    p.m_tiles = (p.tokens - p.m_base + BM - 1) / BM;
    p.n_tiles = (p.width * p.n_out + BN - 1) / BN;
    const unsigned blocks = (unsigned)((int64_t)p.m_tiles * p.n_tiles);
    if (p.d_in % X3_BK == 0) {
        p.chunk = std::max(1, (p.chunk + 1) / 2);  // units of 32 indices
        if (p.xp != nullptr)
            hipLaunchKernelGGL((qkv_proj_x3p<OUT, false>), dim3(blocks), dim3(threads<false>()), (x3p_lds<false>()),
                               stream, p);
        else
            hipLaunchKernelGGL((qkv_proj_x3<OUT, false>), dim3(blocks), dim3(threads<false>()), (x3_lds<false>()),
                               stream, p);
    } else if (p.d_in % 32 == 0)
        hipLaunchKernelGGL((qkv_proj<OUT, 32, false>), dim3(blocks), dim3(threads<false>()), (proj_lds<32, false>()),
                           stream, p);
    else
        hipLaunchKernelGGL((qkv_proj<OUT, 16, false>), dim3(blocks), dim3(threads<false>()), (proj_lds<16, false>()),
                           stream, p);
    return hipGetLastError();
}

template <int OUT>
hipError_t launch_unsplit(ProjParams p, hipStream_t stream) {
    // The token rows from p.m_base on (0 at the first call).
    const int64_t rows = (int64_t)p.tokens - p.m_base;
    const int64_t big_m = (rows + 127) / 128, big_n = (p.width * p.n_out + 127) / 128;
    if (big_m * big_n < kBigTilesMin) return launch_small<OUT>(p, stream);
    if (p.d_in % X3_BK == 0 && p.xp != nullptr && p.splits <= 1 && p.m_base == 0) {
        // Pre-split operands: 256 x 128 tiles, one workgroup per CU, in whole rounds; the token rows
        // past them go to 128 x 128 / 64 x 64 tiles below.
        const int64_t wide_m = rows / kWideM, slots = (int64_t)device_cus();
        const int64_t m_wide = slots > 0 ? (wide_m * big_n - (wide_m * big_n) % slots) / big_n : 0;
        if (m_wide > 0) {
            ProjParams q = p;
            q.m_tiles = (int32_t)m_wide;
            q.n_tiles = (int32_t)big_n;
            q.chunk = std::max(1, (p.chunk + 1) / 2);  // units of 32 indices
            hipLaunchKernelGGL((qkv_proj_x3w<OUT>), dim3((unsigned)(m_wide * big_n)), dim3(512),
                               (size_t)(2 * kWideStage), stream, q);
            if (const hipError_t e = hipGetLastError(); e != hipSuccess || m_wide * kWideM >= rows) return e;
            p.m_base = (int32_t)(m_wide * kWideM);
            return launch_unsplit<OUT>(p, stream);
        }
    }
    if (p.d_in % X3_BK == 0) {
        // The bf16 three-way split, one workgroup per CU: the token tiles past the full rounds go
        // to SMALL tiles when the last round would be less than half full, as below.
        int64_t m_big = big_m;
        const int64_t slots = (int64_t)device_cus(), rest = slots > 0 ? (big_m * big_n) % slots : 0;
        if (slots > 0 && big_m * big_n > slots && rest > 0 && 2 * rest < slots)
            m_big = std::max<int64_t>(1, (big_m * big_n - rest) / big_n);
        ProjParams q = p;
        q.m_tiles = (int32_t)m_big;
        q.n_tiles = (int32_t)big_n;
        q.chunk = std::max(1, (p.chunk + 1) / 2);  // units of 32 indices
        if (q.xp != nullptr)
            hipLaunchKernelGGL((qkv_proj_x3p<OUT, true>), dim3((unsigned)(m_big * big_n)), dim3(threads<true>()),
                               (x3p_lds<true>()), stream, q);
        else
            hipLaunchKernelGGL((qkv_proj_x3<OUT, true>), dim3((unsigned)(m_big * big_n)), dim3(threads<true>()),
                               (x3_lds<true>()), stream, q);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess || m_big * 128 >= rows) return e;
        p.m_base += (int32_t)(m_big * 128);
        return launch_small<OUT>(p, stream);
    }
    // BIG tiles run two per CU, in rounds that each take one tile's time. A last round less than
    // half full would cost a whole one: the token tiles past the full rounds go to SMALL tiles
    // instead (four per CU, a quarter of the work each), in a second launch.
    int64_t m_big = big_m;
    const int64_t slots = 2 * (int64_t)device_cus(), rest = slots > 0 ? (big_m * big_n) % slots : 0;
    if (slots > 0 && big_m * big_n > slots && rest > 0 && 2 * rest < slots)
        m_big = std::max<int64_t>(1, (big_m * big_n - rest) / big_n);
    p.m_tiles = (int32_t)m_big;
    p.n_tiles = (int32_t)big_n;
    // 16-wide steps: with 32-wide ones the eight waves' operands, totals and running chunks need
    // more than the 128 registers that four waves per SIMD leave.
    hipLaunchKernelGGL((qkv_proj<OUT, 16, true>), dim3((unsigned)(m_big * big_n)), dim3(threads<true>()),
                       (proj_lds<16, true>()), stream, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || m_big * 128 >= rows) return e;
    p.m_base += (int32_t)(m_big * 128);
    return launch_small<OUT>(p, stream);
}

}  // namespace

// Accumulation chunk (in 16-wide units) for a workgroup range of `units` units: a chunk's chain is
// 4 c rounded steps and the chunk totals add units / c more, so c ~ sqrt(units / 4) keeps the
// longest run of roundings near its minimum, 2 sqrt(4 units) (28 steps at d_in 768, 12 at 128).
static int proj_chunk(int units) {
    int c = 1;
    while (4 * (c + 1) + (units + c) / (c + 1) < 4 * c + (units + c - 1) / c) c++;
    return c;
}

// Products the 16-token kernel takes (proj_skinny).
static bool skinny(const ProjParams& p) {
    return p.tokens <= kSkinnyTokens && p.d_in <= kSkinnyMaxIn && p.rope_cos == nullptr && p.out_dtype == 0 &&
           p.x_pre == nullptr && p.y_planes == nullptr;
}

bool proj_fuses_input_norm(int64_t tokens, int64_t d_in) {
    return tokens > 0 && tokens <= kSkinnyTokens && d_in > 0 && d_in <= kSkinnyMaxIn && d_in % 16 == 0;
}

size_t proj_split_bytes(ProjParams& p) {
    p.m_tiles = (p.tokens + BM - 1) / BM;
    p.n_tiles = (p.width * p.n_out + BN - 1) / BN;
    const int64_t blocks = (int64_t)p.m_tiles * p.n_tiles;
    const int steps = p.d_in / 16;
    p.splits = 1;
    p.split_steps = steps;
    p.partial = nullptr;
    if (p.x_pre != nullptr || p.y_planes != nullptr) return 0;  // pre-split operands: never split
    // f32 outputs, no RoPE; several outputs only without an epilogue; at most half a launch of
    // tiles (four workgroups per CU), and at least 16 steps to share out.
    if (!((p.n_out == 1 || p.epi == kEpiNone) && p.rope_cos == nullptr && p.out_dtype == 0 && blocks < 512 &&
          steps >= 16) ||
        skinny(p))
        return 0;
    // About 512 workgroups (two per CU): more splits of these short reductions cost more in
    // partial traffic and per-workgroup start-up than they gain in parallelism (measured on the
    // Chronos-Bolt-small forecast: 1.160 ms for about 1024, 1.106 ms for about 512, 1.185 ms for
    // at most two splits).
    int s = (int)std::min<int64_t>((512 + blocks - 1) / blocks, std::min(steps / 8, 16));
    if (s < 2) return 0;
    int per = (steps + s - 1) / s;
    if (p.d_in % X3_BK == 0) per += per & 1;  // whole 32-index steps for the bf16x3 kernel
    s = (steps + per - 1) / per;
    if (s < 2) return 0;
    p.splits = s;
    p.split_steps = per;
    // s * blocks <= 512 + blocks - 1 < 1536 and tokens * width <= blocks * BM * BN, so the partials
    // always fit kSplitWorkspaceBytes.
    return (size_t)s * p.tokens * p.width * p.n_out * sizeof(float);
}

hipError_t launch_proj(const ProjParams& p0, hipStream_t stream) {
    ProjParams p = p0;
    p.m_base = 0;
    if (p.tokens <= 0 || p.width <= 0 || p.n_out <= 0) return hipSuccess;
    if (p.d_in % 16 || p.d_in <= 0 || p.n_out > 4 || p.seq <= 0 || p.out_dtype < 0 || p.out_dtype > 2 ||
        p.w_ld < p.d_in || p.width % 4 || (p.n_out > 1 && p.width % kHeadDim) ||
        (p.rope_cos != nullptr && p.width % kHeadDim) ||
        (p.out_dtype != 0 && (p.epi != kEpiNone || p.alpha != 1.f || p.bias != nullptr)) ||
        (p.bias != nullptr && p.n_out != 1) ||
        (p.norm_scale != nullptr && (p.n_out != 1 || p.out_dtype != 0 || p.norm_out == nullptr || p.y0_batch != 0)) ||
        (p.epi != kEpiNone && (p.y0_batch | p.y1_batch | p.y2_batch | p.y3_batch) != 0) || p.epi < kEpiNone ||
        p.epi > kEpiSilu)
        return hipErrorInvalidValue;
    if ((int64_t)((p.tokens + BM - 1) / BM) * ((p.width * p.n_out + BN - 1) / BN) > 0x7fffffff)
        return hipErrorInvalidValue;
    if (p.in_norm_scale != nullptr && !skinny(p)) return hipErrorInvalidValue;  // the 16-token kernel only
    if (skinny(p)) {
        p.chunk = proj_chunk((p.d_in / 16 + SKW - 1) / SKW);
        hipLaunchKernelGGL(proj_skinny, dim3((unsigned)((p.width * p.n_out + 15) / 16)), dim3(64 * SKW), kSkinnyLds,
                           stream, p);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess && p.norm_scale != nullptr)
            e = launch_rms_norm(static_cast<const float*>(p.y0), p.y0_tok, p.norm_out, p.norm_out_tok, p.norm_scale,
                                p.tokens, p.width, p.norm_eps, stream);
        return e;
    }
    // Pre-split operands when the entry point lent a large enough PlaneWorkspace: the weights split
    // into it, and x too unless its producer split it (x_pre). x_pre / y_planes need that path.
    p.xp = p.wp = nullptr;
    const int64_t n_cols = (int64_t)p.width * p.n_out;
    const bool fused = p.x_pre != nullptr || p.y_planes != nullptr;
    if (fused && (!proj_planes_ready(p.tokens, p.d_in, n_cols) ||
                  (p.y_planes != nullptr && (p.n_out != 1 || p.width % X3_BK || p.out_dtype != 0 || p.rope_cos != nullptr))))
        return hipErrorInvalidValue;
    if (t_plane_ws != nullptr && planes_pay(p.tokens, p.d_in, n_cols)) {
        const size_t xb = p.x_pre != nullptr ? 0 : plane_operand_bytes(p.tokens, p.d_in);
        if (xb + plane_operand_bytes(n_cols, p.d_in) <= t_plane_bytes) {
            const int kc = p.d_in / X3_BK;
            uint8_t* const xp = static_cast<uint8_t*>(t_plane_ws);
            uint8_t* const wp = xp + xb;
            SplitSrc sw = {{p.w0, p.w1 ? p.w1 : p.w0, p.w2 ? p.w2 : p.w0, p.w3 ? p.w3 : p.w0}, p.w_ld, p.width,
                           (int32_t)n_cols, kc};
            if (p.x_pre == nullptr) {
                SplitSrc sx = {{p.x, p.x, p.x, p.x}, p.x_tok, p.tokens, p.tokens, kc};
                const int64_t cx = (int64_t)((p.tokens + 15) / 16) * kc;
                hipLaunchKernelGGL(split_planes, dim3((unsigned)((cx + 3) / 4)), dim3(256), 0, stream, sx, xp);
            }
            const int64_t cw = (n_cols + 15) / 16 * kc;
            hipLaunchKernelGGL(split_planes, dim3((unsigned)((cw + 3) / 4)), dim3(256), 0, stream, sw, wp);
            if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
            p.xp = p.x_pre != nullptr ? p.x_pre : xp;
            p.wp = wp;
        }
    }
    // Small products (a few token tiles: the decoder's 16 rows, short encoders) leave most CUs idle
    // and each workgroup walks the whole reduction; split it over workgroups instead (16-wide
    // steps), with the partial tiles summed in a fixed order by proj_reduce.
    if (const size_t part_bytes = proj_split_bytes(p); part_bytes > 0) {
        // The entry point that queues this product owns the partials' buffer (SplitWorkspace);
        // without one the product is refused rather than run unsplit, which would give other bits.
        // The split rule keeps the partials within the buffer; a rule that did not is refused here,
        // before any kernel could write past it.
        if (t_split_ws == nullptr || part_bytes > kSplitWorkspaceBytes) return hipErrorInvalidValue;
        p.partial = t_split_ws;
    }
    const int64_t blocks = (int64_t)p.m_tiles * p.n_tiles;
    p.chunk = proj_chunk(p.splits > 1 ? p.split_steps : p.d_in / 16);
    if (p.splits > 1) {
        if (p.d_in % X3_BK == 0) {
            ProjParams q = p;
            q.chunk = std::max(1, (p.chunk + 1) / 2);  // units of 32 indices
            if (q.xp != nullptr)
                hipLaunchKernelGGL((qkv_proj_x3p<0, false>), dim3((unsigned)(blocks * p.splits)),
                                   dim3(threads<false>()), (x3p_lds<false>()), stream, q);
            else
                hipLaunchKernelGGL((qkv_proj_x3<0, false>), dim3((unsigned)(blocks * p.splits)),
                                   dim3(threads<false>()), (x3_lds<false>()), stream, q);
        } else {
            hipLaunchKernelGGL((qkv_proj<0, 16, false>), dim3((unsigned)(blocks * p.splits)), dim3(threads<false>()),
                               (proj_lds<16, false>()), stream, p);
        }
        hipError_t e = hipGetLastError();
        if (e == hipSuccess && p.norm_scale != nullptr) {
            hipLaunchKernelGGL(proj_reduce_norm, dim3((unsigned)((p.tokens + 3) / 4)), dim3(256), 0, stream, p);
            e = hipGetLastError();
        } else if (e == hipSuccess) {
            const int64_t n = (int64_t)p.tokens * (p.width * p.n_out / 4);
            hipLaunchKernelGGL(proj_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p);
            e = hipGetLastError();
        }
        return e;
    }
    if (p.norm_scale != nullptr) {
        const hipError_t e = launch_unsplit<0>(p, stream);
        if (e != hipSuccess) return e;
        return launch_rms_norm(static_cast<const float*>(p.y0), p.y0_tok, p.norm_out, p.norm_out_tok, p.norm_scale,
                               p.tokens, p.width, p.norm_eps, stream);
    }
    if (p.out_dtype == 1) return launch_unsplit<1>(p, stream);
    if (p.out_dtype == 2) return launch_unsplit<2>(p, stream);
    return launch_unsplit<0>(p, stream);
}

namespace {
// dst[c][r] = src[r][c] for r < rows, c < cols: 32 x 32 tiles through LDS (one padding column, so
// the column reads of the tile hit 32 different banks); loads and stores are row-contiguous.
__global__ __launch_bounds__(256) void transpose_f32(const float* __restrict__ src, int64_t ld_src,
                                                     float* __restrict__ dst, int64_t ld_dst, int rows, int cols) {
    __shared__ float t[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 8 rows of 32 per pass
#pragma unroll
    for (int i = 0; i < 32; i += 8) {
        const int r = r0 + ty + i, c = c0 + tx;
        if (r < rows && c < cols) t[ty + i][tx] = src[(int64_t)r * ld_src + c];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 32; i += 8) {
        const int c = c0 + ty + i, r = r0 + tx;
        if (c < cols && r < rows) dst[(int64_t)c * ld_dst + r] = t[tx][ty + i];
    }
}
}  // namespace

hipError_t launch_transpose_f32(const float* src, int64_t ld_src, float* dst, int64_t ld_dst, int rows, int cols,
                                hipStream_t stream) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
    hipLaunchKernelGGL(transpose_f32, grid, dim3(256), 0, stream, src, ld_src, dst, ld_dst, rows, cols);
    return hipGetLastError();
}

}  // namespace tsfm
