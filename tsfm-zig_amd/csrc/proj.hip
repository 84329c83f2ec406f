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
// computes a 64-token x 64-column tile (one head) with K = d_in in 32-wide steps (16-wide when
// d_in is not a multiple of 32): x and w tiles go HBM/L2 -> registers -> LDS (double-buffered, one
// barrier per step), and each of the four waves multiplies a 32 x 32 sub-tile with
// v_mfma_f32_16x16x4_f32 in four accumulation chains, the weight rows as the A operand so that each
// lane ends with four consecutive output columns of one token (16-byte stores, and the RoPE
// partner column i + 32 in the same lane); f32 outputs, or bf16/f16 for the half-precision
// attention path. Four workgroups share a CU (one wave of each per SIMD), so one's step barrier
// and prologue are covered by the others' products.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

constexpr int BM = 64;           // tokens per workgroup tile
constexpr int BN = 64;           // output columns per workgroup tile: one head
constexpr int NT = 256;          // four waves: 2 (32 tokens) x 2 (column pairs)
constexpr int GM = 8;            // token tiles that sweep the column tiles together
// Reduction step BK (16 or 32; 32 when d_in allows): LDS rows padded to BK + 4 floats, so the 16
// rows one operand read touches hit distinct banks.
template <int BK>
constexpr size_t proj_lds() { return (size_t)2 * (BM + BN) * (BK + 4) * sizeof(float); }
static_assert(kSplitWorkspaceBytes == (size_t)1536 * BM * BN * sizeof(float), "split workspace size");

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
//
// Accumulation order. v_mfma_f32_16x16x4_f32 rounds as it accumulates, so one accumulator carried
// across the whole reduction would be a single chain of d_in rounded additions, several times the
// error of the reference's nn.lanes vector partial sums (src/core/nn.zig:68-126: 8 or 16 lanes,
// then a reduction). Each wave therefore keeps four accumulators per output block, one per
// instruction slot j of a 16-wide chunk (reduction indices 16c + 4g + j), and sums them as a tree
// at the end: four independent chains of d_in / 4 products, like a 4-lane reference, in a fixed
// order. Waves of 32 tokens x 32 columns hold the four chains in 64 registers per lane.
template <int OUT, int BK>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4, 4))) void qkv_proj(ProjParams p) {
    constexpr int LDS_ROW = BK + 4;
    constexpr int NX = BM * BK / 4, NW = BN * BK / 4;  // float4s of the x and weight tiles per step
    constexpr int PER = (NX + NW + NT - 1) / NT;       // float4s a thread stages per step (at most)
    static_assert(NX % 64 == 0 && (NX + NW) % 64 == 0, "loader slots are whole waves");
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* const xs = smem;                          // [2][BM][LDS_ROW]
    float* const ws = smem + 2 * BM * LDS_ROW;       // [2][BN][LDS_ROW]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tm, tn;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int split = p.splits > 1 ? logical % p.splits : 0;  // this workgroup's share of the reduction
    tile_of(p.splits > 1 ? logical / p.splits : logical, p.m_tiles, p.n_tiles, tm, tn);
    const int n_cols = p.width * p.n_out;

    // Loader: slot f = tid + NT i (i < PER) of a step is float4 f of the x tile (f < NX) or float4
    // f - NX of the weight tile (f < NX + NW); slots past that are idle (whole waves). A tile's
    // float4 e is row e / (BK / 4), columns 4 (e % (BK / 4)) .. + 3. Rows past the end are clamped
    // to the last row: they feed only outputs that are not stored.
    const float* src[PER];
    float* dst[PER];
    int stage[PER];  // floats between the two LDS buffers of this slot's tile; 0 = idle slot
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int f = tid + NT * i;
        const bool is_x = f < NX;
        const int e = is_x ? f : min(f - NX, NW - 1), lr = e / (BK / 4), lc = (e % (BK / 4)) * 4;
        if (is_x) {
            src[i] = p.x + (int64_t)min(tm * BM + lr, p.tokens - 1) * p.x_tok + lc;
        } else {
            const int n = min(tn * BN + lr, n_cols - 1);
            const int sel = n / p.width;
            const float* w = sel == 0 ? p.w0 : sel == 1 ? p.w1 : sel == 2 ? p.w2 : p.w3;
            src[i] = w + (int64_t)(n - sel * p.width) * p.w_ld + lc;
        }
        dst[i] = (is_x ? xs : ws) + lr * LDS_ROW + lc;
        stage[i] = f < NX + NW ? (is_x ? BM : BN) * LDS_ROW : 0;
    }

    // Wave layout: token block wm (32 tokens), column pair wq: the wave's two 16-column blocks are wq
    // and wq + 2 of the workgroup's head, so a RoPE pair (i, i + 32) is in one lane.
    // Operand reads: lane l takes row (l & 15) of a 16-row block and the four reduction indices
    // 4 (l >> 4) .. + 3 of a 16-wide chunk; matrix instruction j uses element j, the same reduction
    // index on both operands.
    const int wm = wave & 1, wq = wave >> 1;
    const float* const xr = xs + (wm * 32 + (lane & 15)) * LDS_ROW + 4 * (lane >> 4);
    const float* const wr = ws + (16 * wq + (lane & 15)) * LDS_ROW + 4 * (lane >> 4);

    f32x4 acc[4][2][2];  // [chain j][column block wq, wq + 2][token block]: columns 4 (l >> 4) + r, token l & 15
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < 2; b++) acc[j][a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int t0 = split * p.split_steps;
    const int steps = p.splits > 1 ? min(p.d_in / BK, t0 + p.split_steps) : p.d_in / BK;
    f32x4 rv[PER];
#pragma unroll
    for (int i = 0; i < PER; i++)
        if (stage[i]) rv[i] = ld4(src[i] + t0 * BK);
#pragma unroll
    for (int i = 0; i < PER; i++)
        if (stage[i]) st4(dst[i], rv[i]);
    __syncthreads();
    for (int t = t0; t < steps; t++) {
        const int buf = (t - t0) & 1;
        if (t + 1 < steps) {
#pragma unroll
            for (int i = 0; i < PER; i++)
                if (stage[i]) rv[i] = ld4(src[i] + (t + 1) * BK);
        }
        // Operands of chunk c + 1 are read from LDS while chunk c's products run.
        f32x4 wa[2], xb[2];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            wa[b] = ld4(wr + (buf * BN + 32 * b) * LDS_ROW);
            xb[b] = ld4(xr + (buf * BM + 16 * b) * LDS_ROW);
        }
#pragma unroll
        for (int c = 0; c < BK / 16; c++) {
            f32x4 wn_[2], xn_[2];
            if (c + 1 < BK / 16) {
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    wn_[b] = ld4(wr + (buf * BN + 32 * b) * LDS_ROW + 16 * (c + 1));
                    xn_[b] = ld4(xr + (buf * BM + 16 * b) * LDS_ROW + 16 * (c + 1));
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
#pragma unroll
                    for (int mb = 0; mb < 2; mb++)
                        acc[j][nb][mb] =
                            __builtin_amdgcn_mfma_f32_16x16x4f32(wa[nb][j], xb[mb][j], acc[j][nb][mb], 0, 0, 0);
            if (c + 1 < BK / 16) {
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    wa[b] = wn_[b];
                    xb[b] = xn_[b];
                }
            }
        }
        // The other buffer was last read in step t - 1, which every wave has left (barrier below).
        if (t + 1 < steps) {
#pragma unroll
            for (int i = 0; i < PER; i++)
                if (stage[i]) st4(dst[i] + (buf ^ 1) * stage[i], rv[i]);
        }
        __syncthreads();
    }
    f32x4 sum[2][2];
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
#pragma unroll
        for (int mb = 0; mb < 2; mb++) sum[nb][mb] = (acc[0][nb][mb] + acc[1][nb][mb]) + (acc[2][nb][mb] + acc[3][nb][mb]);

    // Epilogue: this wave's columns are blocks wq and wq + 2 of one head of one output (or, with one
    // output of a width that is not a multiple of 64, columns of a partial head: groups of four
    // columns past the width are not stored).
    const int n0 = tn * BN;
    if (n0 >= n_cols) return;
    const int sel = n0 / p.width, col = n0 - sel * p.width;
    const int cq = 16 * wq + 4 * (lane >> 4);  // this lane's first column of block wq in the head
    if (p.splits > 1) {  // partial sums only; proj_reduce adds them up in split order and finishes
        // Partial row m of split s holds all n_cols columns (every output side by side).
#pragma unroll
        for (int mb = 0; mb < 2; mb++) {
            const int m = tm * BM + wm * 32 + mb * 16 + (lane & 15);
            if (m >= p.tokens) continue;
            float* const out = p.partial + ((int64_t)split * p.tokens + m) * n_cols + n0 + cq;
#pragma unroll
            for (int nb = 0; nb < 2; nb++)
                if (col + cq + 32 * nb < p.width) st4(out + 32 * nb, sum[nb][mb]);
        }
        return;
    }
    void* const y = sel == 0 ? p.y0 : sel == 1 ? p.y1 : sel == 2 ? p.y2 : p.y3;
    const bool rope = p.rope_cos != nullptr && sel < 2;
#pragma unroll
    for (int mb = 0; mb < 2; mb++) {
        const int m = tm * BM + wm * 32 + mb * 16 + (lane & 15);
        if (m >= p.tokens) continue;
        if (p.alpha != 1.f) {  // gemmNT's alpha, applied to the finished sum (src/core/nn.zig:100)
#pragma unroll
            for (int nb = 0; nb < 2; nb++) sum[nb][mb] *= p.alpha;
        }
        if (rope) {
            // Token t of series row b: row t of table (rope_row0 + b) / rope_rows_per_table.
            const int b = m / p.seq, tok = m - b * p.seq;
            const int table = p.rope_rows_per_table > 0 ? (p.rope_row0 + b) / p.rope_rows_per_table : 0;
            const int64_t at = (int64_t)table * p.rope_table_stride + (int64_t)tok * (kHeadDim / 2) + cq;
            rope4(sum[0][mb], sum[1][mb], ld4(p.rope_cos + at), ld4(p.rope_sin + at));
        }
        const int64_t at = out_offset(p, sel, m) + col + cq;
        if constexpr (OUT == 0) {
            float* const out = static_cast<float*>(y) + at;
            const float* const res = p.epi == kEpiResidual ? p.resid + (int64_t)m * p.resid_tok + col + cq : nullptr;
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                if (col + cq + 32 * nb >= p.width) continue;
                f32x4 v = sum[nb][mb];
                if (p.bias != nullptr) v = v + ld4(p.bias + col + cq + 32 * nb);  // nn.linear's bias (linearCols, nn.zig:254)
                if (p.epi == kEpiResidual) v = ld4(res + 32 * nb) + v;  // x + delta, one rounding
                else v = epi_act(p.epi, v);
                st4(out + 32 * nb, v);
            }
        } else {
            uint16_t* const out = static_cast<uint16_t*>(y) + at;
#pragma unroll
            for (int nb = 0; nb < 2; nb++) {
                const f32x4 v = sum[nb][mb];
                *reinterpret_cast<u32x2*>(out + 32 * nb) = u32x2{pack2<OUT == 1>(v[0], v[1]), pack2<OUT == 1>(v[2], v[3])};
            }
        }
    }
}

// Sum of the split partials in split order (deterministic), then the epilogue: alpha, and with one
// output bias, ReLU or residual; f32 store into the output the column belongs to. One thread per
// four columns of a token (width is a multiple of 4, so a group never straddles two outputs).
__global__ __launch_bounds__(256) void proj_reduce(ProjParams p) {
    const int n_cols = p.width * p.n_out, q = n_cols / 4;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.tokens * q) return;
    const int m = (int)(idx / q), c = (int)(idx % q) * 4;
    f32x4 v = ld4(p.partial + (int64_t)m * n_cols + c);
    for (int s = 1; s < p.splits; s++) v = v + ld4(p.partial + ((int64_t)s * p.tokens + m) * n_cols + c);
    if (p.alpha != 1.f) v *= p.alpha;
    const int sel = c / p.width, col = c - sel * p.width;
    if (p.bias != nullptr) v = v + ld4(p.bias + col);
    if (p.epi == kEpiResidual) v = ld4(p.resid + (int64_t)m * p.resid_tok + col) + v;
    else v = epi_act(p.epi, v);
    float* const y = static_cast<float*>(sel == 0 ? p.y0 : sel == 1 ? p.y1 : sel == 2 ? p.y2 : p.y3);
    st4(y + out_offset(p, sel, m) + col, v);
}

// proj_reduce for one output followed by the row norm of the finished rows: one wave per token
// row sums the partials of its four-column groups in split order, applies the epilogue, stores
// y0, and keeps the row's sum of squares; then norm_out = y0 * inv * norm_scale. The row norm's
// grouping and order are rms_norm_rows', so the result has the same bits as the two launches.
__global__ __launch_bounds__(256) void proj_reduce_norm(ProjParams p) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= p.tokens) return;
    const int W = p.width;
    float* const y = static_cast<float*>(p.y0) + out_offset(p, 0, row);
    float ss = 0.f;
    for (int c = 4 * lane; c < W; c += 256) {
        f32x4 v = ld4(p.partial + (int64_t)row * W + c);
        for (int s = 1; s < p.splits; s++) v = v + ld4(p.partial + ((int64_t)s * p.tokens + row) * W + c);
        if (p.alpha != 1.f) v *= p.alpha;
        if (p.bias != nullptr) v = v + ld4(p.bias + c);
        if (p.epi == kEpiResidual) v = ld4(p.resid + (int64_t)row * p.resid_tok + c) + v;
        else v = epi_act(p.epi, v);
        st4(y + c, v);
        ss = sumsq4(ss, v);
    }
    const float inv = rms_inv(ss, W, p.norm_eps);
    float* const o = p.norm_out + (int64_t)row * p.norm_out_tok;
    for (int c = 4 * lane; c < W; c += 256) st4(o + c, rms_apply(ld4(y + c), inv, ld4(p.norm_scale + c)));
}

}  // namespace

namespace {

// The split-partials buffer of the calling thread's current library call (SplitWorkspace).
thread_local float* t_split_ws = nullptr;

}  // namespace

SplitWorkspace::SplitWorkspace(float* buf) : prev_(t_split_ws) { t_split_ws = buf; }
SplitWorkspace::~SplitWorkspace() { t_split_ws = prev_; }

namespace {

// The unsplit product: 32-wide steps when d_in allows (half the step barriers), else 16-wide. The
// chains are the same either way (chain j sums reduction indices 16c + 4g + j in increasing c), so
// the result does not depend on the step width.
template <int OUT>
hipError_t launch_unsplit(const ProjParams& p, int64_t blocks, hipStream_t stream) {
    if (p.d_in % 32 == 0)
        hipLaunchKernelGGL((qkv_proj<OUT, 32>), dim3((unsigned)blocks), dim3(NT), proj_lds<32>(), stream, p);
    else
        hipLaunchKernelGGL((qkv_proj<OUT, 16>), dim3((unsigned)blocks), dim3(NT), proj_lds<16>(), stream, p);
    return hipGetLastError();
}

}  // namespace

size_t proj_split_bytes(ProjParams& p) {
    p.m_tiles = (p.tokens + BM - 1) / BM;
    p.n_tiles = (p.width * p.n_out + BN - 1) / BN;
    const int64_t blocks = (int64_t)p.m_tiles * p.n_tiles;
    const int steps = p.d_in / 16;
    p.splits = 1;
    p.split_steps = steps;
    p.partial = nullptr;
    // f32 outputs, no RoPE; several outputs only without an epilogue; at most half a launch of
    // tiles (four workgroups per CU), and at least 16 steps to share out.
    if (!((p.n_out == 1 || p.epi == kEpiNone) && p.rope_cos == nullptr && p.out_dtype == 0 && blocks < 512 &&
          steps >= 16))
        return 0;
    int s = (int)std::min<int64_t>((1024 + blocks - 1) / blocks, std::min(steps / 8, 16));
    if (s < 2) return 0;
    const int per = (steps + s - 1) / s;
    s = (steps + per - 1) / per;
    p.splits = s;
    p.split_steps = per;
    // s * blocks <= 1024 + blocks - 1 < 1536 and tokens * width <= blocks * BM * BN, so the partials
    // always fit kSplitWorkspaceBytes.
    return (size_t)s * p.tokens * p.width * p.n_out * sizeof(float);
}

hipError_t launch_proj(const ProjParams& p0, hipStream_t stream) {
    ProjParams p = p0;
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
    // Small products (a few token tiles: the decoder's 16 rows, short encoders) leave most CUs idle
    // and each workgroup walks the whole reduction; split it over workgroups instead (16-wide
    // steps), with the partial tiles summed in a fixed order by proj_reduce.
    if (proj_split_bytes(p) > 0) {
        // The entry point that queues this product owns the partials' buffer (SplitWorkspace);
        // without one the product is refused rather than run unsplit, which would give other bits.
        if (t_split_ws == nullptr) return hipErrorInvalidValue;
        p.partial = t_split_ws;
    }
    const int64_t blocks = (int64_t)p.m_tiles * p.n_tiles;
    if (p.splits > 1) {
        hipLaunchKernelGGL((qkv_proj<0, 16>), dim3((unsigned)(blocks * p.splits)), dim3(NT), proj_lds<16>(), stream, p);
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
        const hipError_t e = launch_unsplit<0>(p, blocks, stream);
        if (e != hipSuccess) return e;
        return launch_rms_norm(static_cast<const float*>(p.y0), p.y0_tok, p.norm_out, p.norm_out_tok, p.norm_scale,
                               p.tokens, p.width, p.norm_eps, stream);
    }
    if (p.out_dtype == 1) return launch_unsplit<1>(p, blocks, stream);
    if (p.out_dtype == 2) return launch_unsplit<2>(p, blocks, stream);
    return launch_unsplit<0>(p, blocks, stream);
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
