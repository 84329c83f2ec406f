// Timestral variate attention on the matrix cores (gfx950).
//
// The reference's VariateJob.run (src/timestral/model.zig:648-709): at every (series group g,
// token slot t) the vall rows of the group attend each other, per head, through a vall x vall
// allowed matrix (diagonal always open; key validity on encoder slots; the covariate firewalls).
// Up to 16 rows, one wave takes one (g, t) and a block of heads (a workgroup, every head block of
// one (g, t)): with vall rows per head, 16 / vall heads share one 16 x 16 score block (slot s =
// head-in-block * vall + row), so one set of v_mfma_f32_16x16x4_f32 serves several heads; scores
// between different heads are masked out. More rows (up to kVariateMaxRows): a wave takes one head
// and 16 query rows and walks the keys in 16-row blocks with an online softmax (the same products
// per block; O and the row sums rescaled when a block raises the row max).
//
//   S^T = K . Q^T   16 key slots x 16 query slots over the 64 head dims: 16 instructions in four
//                   accumulation chains summed as a tree (as in attn_f32.hip); q pre-scaled.
//   softmax         per query slot over the four 16-lane groups (max4 / sum4), exp2-based.
//   O^T += V^T P^T  4 key steps x 4 dim blocks, P straight from the S^T accumulator.
//
// Operands come straight from HBM (each (g, t) is read once), through one buffer descriptor over
// the token's rows: q and k as 16-byte loads of the lane's dims, v as 4-byte loads of 16
// consecutive dims. An optional gate multiplies the result by sigmoid(gate) before the store
// (nn.mulSigmoid, src/core/nn.zig:423-433, fused; the reciprocal is v_rcp_f32, within 1 ulp of the
// reference's division).
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

// One head block of one (group, token) item.
__device__ __forceinline__ void variate_block(const VariateParams& p, int item, int blk, int lane) {
#pragma clang fp contract(off)
    const int ql = lane & 15, g = lane >> 4;
    const int vall = p.vall;
    const int grp = item / p.n_tok, tok = item % p.n_tok;
    const int h0 = blk * p.heads_per_block;
    const int heads_here = min(p.heads_per_block, p.heads - h0);
    const int live = heads_here * vall;  // valid slots of this block
    const int64_t r0 = (int64_t)grp * vall;
    const int dm = p.heads * kHeadDim;  // d_model: offset of k, and 2 * dm of v, in a token's qkv

    // Slot s < 16 of the block: head h0 + s / vall, row s % vall. s / vall by a multiply and a
    // shift (exact for s < 16 with the rounded-up 16-bit reciprocal).
    const uint32_t rcp = (65536u + (uint32_t)vall - 1u) / (uint32_t)vall;
    auto sdiv = [&](int s) { return (int)(((uint32_t)s * rcp) >> 16); };

    // The vall rows of this token, through one buffer descriptor: a slot's byte offset is
    // row * qkv_row + part * dm + head * 64 (+ dims); offsets of slots past `live` are pushed out of
    // range, where loads return 0 (no branch, no exec mask).
    const float* tokq = p.qkv + r0 * p.qkv_row + (int64_t)tok * p.qkv_tok;
    const __amdgpu_buffer_rsrc_t qb = make_buf(tokq, p.qkv_span_bytes);
    auto slot_off = [&](int s, int part) -> uint32_t {
        const int hs = sdiv(s), row = s - hs * vall;
        const uint32_t off = (uint32_t)(row * p.qkv_row + part * dm + (h0 + hs) * kHeadDim) * 4u;
        return s < live ? off : 0x80000000u;
    };

    // ---- operands of S^T: lane (ql, g) holds dims 8g..8g+7 and 32+8g..32+8g+7 of query slot ql
    //      (B operand) and of key slot ql (A operand) ----
    const uint32_t qo = slot_off(ql, 0) + 32u * g, ko = slot_off(ql, 1) + 32u * g;
    f32x4 qv[4], kv[4];
    qv[0] = bld4(qb, qo);
    qv[1] = bld4(qb, qo + 16u);
    qv[2] = bld4(qb, qo + 128u);
    qv[3] = bld4(qb, qo + 144u);
    kv[0] = bld4(qb, ko);
    kv[1] = bld4(qb, ko + 16u);
    kv[2] = bld4(qb, ko + 128u);
    kv[3] = bld4(qb, ko + 144u);
    // ---- V^T operand: lane (i = ql, g) takes dim 16db + i of key slot 4g + r ----
    float vv[4][4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t vo = slot_off(4 * g + r, 2) + 4u * ql;
#pragma unroll
        for (int db = 0; db < 4; db++) vv[r][db] = bld1(qb, vo + 64u * db);
    }

    // ---- allowed(query slot ql, key slot 4g + r) ----
    const bool row_ok = ql < live;
    const int hq = sdiv(ql), iq = ql - hq * vall;
    auto role = [&](int i) { return (int)((p.roles[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    const int role_q = role(iq);
    bool allow[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int s = 4 * g + r, hs = sdiv(s), ik = s - hs * vall;
        bool ok = row_ok && s < live && hs == hq;
        if (ik != iq) {
            bool valid = true;
            if (tok < p.n_enc) valid = p.key_valid[(r0 + ik) * p.kv_row + tok] != 0;
            bool forbidden = false;
            if (p.cov) {
                const int role_k = role(ik);
                forbidden = (role_q != kRoleTarget && role_k == kRoleTarget) ||
                            (role_q == kRoleKnown && role_k != kRoleKnown);
            }
            ok = ok && valid && !forbidden;
        }
        allow[r] = ok;
    }

    // ---- S^T = K . Q^T ----
#pragma unroll
    for (int t = 0; t < 4; t++) qv[t] *= p.scale;
    f32x4 c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][0], qv[t][0], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][1], qv[t][1], c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][2], qv[t][2], c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][3], qv[t][3], c3, 0, 0, 0);
    }
    f32x4 sc = (c0 + c1) + (c2 + c3);

    // ---- softmax over the query slot's allowed key slots (the diagonal is one of them) ----
    float mloc = kNegInf;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sc[r] = allow[r] ? sc[r] : kNegInf;
        mloc = fmaxf(mloc, sc[r]);
    }
    const float m = max4(mloc);
    const float m_use = m == kNegInf ? 0.f : m;  // an empty query slot: every weight 0
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        sc[r] = __builtin_amdgcn_exp2f((sc[r] - m_use) * kLog2e);
        lsum += sc[r];
    }
    const float l = sum4(lsum);

    // ---- O^T += V^T . P^T ----
    f32x4 o[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int db = 0; db < 4; db++) o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r][db], sc[r], o[db], 0, 0, 0);

    // ---- normalise, gate, store: lane holds query slot ql, dims 16db + 4g + r ----
    if (!row_ok) return;  // a lane with no query slot is done with this block
    const float inv = 1.0f / l;
    const int head = h0 + hq;
    float* dst = p.o + (r0 + iq) * p.o_row + (int64_t)tok * p.o_tok + head * kHeadDim + 4 * g;
    const float* gp = p.gate ? p.gate + (r0 + iq) * p.gate_row + (int64_t)tok * p.gate_tok + head * kHeadDim + 4 * g
                             : nullptr;
#pragma unroll
    for (int db = 0; db < 4; db++) {
        f32x4 x = o[db] * inv;
        if (gp) {
            const f32x4 gv = ld4(gp + 16 * db);
#pragma unroll
            for (int r = 0; r < 4; r++) x[r] = x[r] * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gv[r] * kLog2e));
        }
        st4(dst + 16 * db, x);
    }
}

// vall > 16: task = (head, block of 16 query rows) of one (group, token) item. Lane (ql, g) holds
// query row 16 qb + ql and, per key block kb, key rows 16 kb + 4g + r (r < 4).
__device__ __forceinline__ void variate_rows(const VariateParams& p, int item, int task, int lane) {
#pragma clang fp contract(off)
    const int ql = lane & 15, g = lane >> 4;
    const int vall = p.vall, nqb = (vall + 15) >> 4;
    const int head = task / nqb, qb = task - head * nqb;
    const int grp = item / p.n_tok, tok = item % p.n_tok;
    const int64_t r0 = (int64_t)grp * vall;
    const int dm = p.heads * kHeadDim;
    const float* tokq = p.qkv + r0 * p.qkv_row + (int64_t)tok * p.qkv_tok;
    const __amdgpu_buffer_rsrc_t rb = make_buf(tokq, p.qkv_span_bytes);
    // Rows past vall are pushed out of the buffer's range: their loads return 0.
    auto row_off = [&](int row, int part) -> uint32_t {
        const uint32_t off = (uint32_t)(row * p.qkv_row + part * dm + head * kHeadDim) * 4u;
        return row < vall ? off : 0x80000000u;
    };
    auto role = [&](int i) { return (int)((p.roles[i >> 2] >> (8 * (i & 3))) & 0xffu); };

    const int iq = 16 * qb + ql;
    const bool row_ok = iq < vall;
    const int role_q = role(min(iq, vall - 1));
    const uint32_t qo = row_off(iq, 0) + 32u * g;
    f32x4 qv[4] = {bld4(rb, qo), bld4(rb, qo + 16u), bld4(rb, qo + 128u), bld4(rb, qo + 144u)};
#pragma unroll
    for (int t = 0; t < 4; t++) qv[t] *= p.scale;

    float m = kNegInf, lsum = 0.f;
    f32x4 o[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
    for (int kb = 0; kb < nqb; kb++) {
        const uint32_t ko = row_off(16 * kb + ql, 1) + 32u * g;
        const f32x4 kv[4] = {bld4(rb, ko), bld4(rb, ko + 16u), bld4(rb, ko + 128u), bld4(rb, ko + 144u)};
        float vv[4][4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t vo = row_off(16 * kb + 4 * g + r, 2) + 4u * ql;
#pragma unroll
            for (int db = 0; db < 4; db++) vv[r][db] = bld1(rb, vo + 64u * db);
        }
        bool allow[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int ik = 16 * kb + 4 * g + r;
            bool ok = row_ok && ik < vall;
            if (ok && ik != iq) {
                if (tok < p.n_enc) ok = p.key_valid[(r0 + ik) * p.kv_row + tok] != 0;
                if (p.cov) {
                    const int role_k = role(ik);
                    ok = ok && !((role_q != kRoleTarget && role_k == kRoleTarget) ||
                                 (role_q == kRoleKnown && role_k != kRoleKnown));
                }
            }
            allow[r] = ok;
        }

        f32x4 c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][0], qv[t][0], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][1], qv[t][1], c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][2], qv[t][2], c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[t][3], qv[t][3], c3, 0, 0, 0);
        }
        f32x4 sc = (c0 + c1) + (c2 + c3);

        float mloc = kNegInf;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sc[r] = allow[r] ? sc[r] : kNegInf;
            mloc = fmaxf(mloc, sc[r]);
        }
        const float mn = fmaxf(m, max4(mloc));
        const float m_use = mn == kNegInf ? 0.f : mn;  // no allowed key yet: every weight 0
        // Earlier blocks' weights were taken against m <= m_use (none yet when m is -inf).
        const float alpha = m == kNegInf ? 0.f : __builtin_amdgcn_exp2f((m - m_use) * kLog2e);
        lsum *= alpha;
#pragma unroll
        for (int db = 0; db < 4; db++) o[db] *= alpha;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sc[r] = __builtin_amdgcn_exp2f((sc[r] - m_use) * kLog2e);
            lsum += sc[r];
        }
        m = mn;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int db = 0; db < 4; db++) o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r][db], sc[r], o[db], 0, 0, 0);
    }
    const float l = sum4(lsum);

    if (!row_ok) return;
    const float inv = 1.0f / l;
    float* dst = p.o + (r0 + iq) * p.o_row + (int64_t)tok * p.o_tok + head * kHeadDim + 4 * g;
    const float* gp = p.gate ? p.gate + (r0 + iq) * p.gate_row + (int64_t)tok * p.gate_tok + head * kHeadDim + 4 * g
                             : nullptr;
#pragma unroll
    for (int db = 0; db < 4; db++) {
        f32x4 x = o[db] * inv;
        if (gp) {
            const f32x4 gv = ld4(gp + 16 * db);
#pragma unroll
            for (int r = 0; r < 4; r++) x[r] = x[r] * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gv[r] * kLog2e));
        }
        st4(dst + 16 * db, x);
    }
}

// One workgroup per (group, token) item: its waves take the item's head blocks, so the rows of
// the token are read by one CU at once.
__global__ __launch_bounds__(256) void variate_attend(VariateParams p) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int blk = wave; blk < p.nblk; blk += 4) variate_block(p, blockIdx.x, blk, lane);
}
__global__ __launch_bounds__(256) void variate_attend_rows(VariateParams p) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int task = wave; task < p.nblk; task += 4) variate_rows(p, blockIdx.x, task, lane);
}

}  // namespace

hipError_t launch_variate(const VariateParams& p0, hipStream_t stream) {
    VariateParams p = p0;
    if (p.vall < 1 || p.vall > kVariateMaxRows || p.heads < 1) return hipErrorInvalidValue;
    const bool rows = p.vall > 16;  // one head and 16 query rows per task
    if (rows) {
        p.heads_per_block = 1;
        p.nblk = p.heads * ((p.vall + 15) / 16);
    } else {
        p.heads_per_block = 16 / p.vall;
        if (p.heads_per_block > p.heads) p.heads_per_block = p.heads;
        p.nblk = (p.heads + p.heads_per_block - 1) / p.heads_per_block;
    }
    const int64_t blocks = (int64_t)p.groups * p.n_tok;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    // One token's vall rows through a 32-bit buffer range (offsets past it read as 0).
    const int64_t span = ((int64_t)(p.vall - 1) * p.qkv_row + 3 * p.heads * kHeadDim) * 4;
    if (span >= 0x80000000LL) return hipErrorNotSupported;
    p.qkv_span_bytes = (uint32_t)span;
    if (rows) hipLaunchKernelGGL(variate_attend_rows, dim3((unsigned)blocks), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(variate_attend, dim3((unsigned)blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace tsfm
