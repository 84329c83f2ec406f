// Timestral variate attention on the matrix cores (gfx950).
//
// The reference's VariateJob.run (src/timestral/model.zig:648-709): at every (series group g,
// token slot t) the vall rows of the group attend each other, per head, through a vall x vall
// allowed matrix (diagonal always open; key validity on encoder slots; the covariate firewalls).
// Here one wave takes one (g, t) and a block of heads: with vall rows per head, 16 / vall heads
// share one 16 x 16 score block (slot s = head-in-block * vall + row), so one set of
// v_mfma_f32_16x16x4_f32 serves several heads; scores between different heads are masked out.
//
//   S^T = K . Q^T   16 key slots x 16 query slots over the 64 head dims: 16 instructions in four
//                   accumulation chains summed as a tree (as in attn_f32.hip); q pre-scaled.
//   softmax         per query slot over the four 16-lane groups (max4 / sum4), exp2-based.
//   O^T += V^T P^T  4 key steps x 4 dim blocks, P straight from the S^T accumulator.
//
// Operands come straight from HBM (each (g, t) is read once): q and k as 16-byte loads of the
// lane's dims, v as 4-byte loads of 16 consecutive dims. An optional gate multiplies the result by
// sigmoid(gate) before the store (nn.mulSigmoid, src/core/nn.zig:423-433, fused).
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

__global__ __launch_bounds__(64) void variate_attend(VariateParams p) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x, ql = lane & 15, g = lane >> 4;
    const int vall = p.vall, slots = p.heads_per_block * vall;
    const int64_t bid = blockIdx.x;
    const int blk = (int)(bid % p.nblk);
    const int64_t item = bid / p.nblk;
    const int grp = (int)(item / p.n_tok), tok = (int)(item % p.n_tok);
    const int h0 = blk * p.heads_per_block;
    const int64_t r0 = (int64_t)grp * vall;
    const int dm = p.heads * kHeadDim;  // d_model: offset of k, and 2 * dm of v, in a token's qkv
    const float* __restrict__ tokq = p.qkv + r0 * p.qkv_row + (int64_t)tok * p.qkv_tok;

    // Slot s of the block: head h0 + s / vall, row s % vall; valid while s < slots and the head
    // exists (the last block may hold fewer heads).
    auto slot_ok = [&](int s) { return s < slots && h0 + s / vall < p.heads; };
    auto slot_ptr = [&](int s, int part) {
        return tokq + (int64_t)(s % vall) * p.qkv_row + part * dm + (h0 + s / vall) * kHeadDim;
    };

    // ---- operands of S^T: lane (ql, g) holds dims 8g..8g+7 and 32+8g..32+8g+7 of query slot ql
    //      (B operand) and of key slot ql (A operand) ----
    const bool row_ok = slot_ok(ql);
    f32x4 qv[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
    f32x4 kv[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
    if (row_ok) {
        const float* qs = slot_ptr(ql, 0) + 8 * g;
        const float* ks = slot_ptr(ql, 1) + 8 * g;
        qv[0] = ld4(qs);
        qv[1] = ld4(qs + 4);
        qv[2] = ld4(qs + 32);
        qv[3] = ld4(qs + 36);
        kv[0] = ld4(ks);
        kv[1] = ld4(ks + 4);
        kv[2] = ld4(ks + 32);
        kv[3] = ld4(ks + 36);
    }
    // ---- V^T operand: lane (i = ql, g) takes dim 16db + i of key slot 4g + r ----
    float vv[4][4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int s = 4 * g + r;
        const bool ok = slot_ok(s);
        const float* vs = slot_ptr(ok ? s : 0, 2) + ql;
#pragma unroll
        for (int db = 0; db < 4; db++) vv[r][db] = ok ? vs[16 * db] : 0.f;
    }

    // ---- allowed(query slot ql, key slot 4g + r) ----
    const int hq = ql / vall, iq = ql % vall;
    auto role = [&](int i) { return (int)((p.roles[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    const int role_q = role(iq);
    bool allow[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int s = 4 * g + r, ik = s % vall;
        bool ok = row_ok && slot_ok(s) && s / vall == hq;
        if (ok && ik != iq) {
            const bool valid = tok >= p.n_enc || p.key_valid[(r0 + ik) * p.kv_row + tok] != 0;
            bool forbidden = false;
            if (p.cov) {
                const int role_k = role(ik);
                forbidden = (role_q != kRoleTarget && role_k == kRoleTarget) ||
                            (role_q == kRoleKnown && role_k != kRoleKnown);
            }
            ok = valid && !forbidden;
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
    f32x4 s = (c0 + c1) + (c2 + c3);

    // ---- softmax over the query slot's allowed key slots (the diagonal is one of them) ----
    float mloc = kNegInf;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        s[r] = allow[r] ? s[r] : kNegInf;
        mloc = fmaxf(mloc, s[r]);
    }
    const float m = max4(mloc);
    const float m_use = m == kNegInf ? 0.f : m;  // an empty query slot: every weight 0
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        s[r] = __builtin_amdgcn_exp2f((s[r] - m_use) * kLog2e);
        lsum += s[r];
    }
    const float l = sum4(lsum);

    // ---- O^T += V^T . P^T ----
    f32x4 o[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int db = 0; db < 4; db++) o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r][db], s[r], o[db], 0, 0, 0);

    // ---- normalise, gate, store: lane holds query slot ql, dims 16db + 4g + r ----
    if (!row_ok) return;
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
            for (int r = 0; r < 4; r++) x[r] = x[r] / (1.0f + __builtin_amdgcn_exp2f(-gv[r] * kLog2e));
        }
        st4(dst + 16 * db, x);
    }
}

}  // namespace

hipError_t launch_variate(const VariateParams& p0, hipStream_t stream) {
    VariateParams p = p0;
    if (p.vall < 1 || p.vall > 16 || p.heads < 1) return hipErrorInvalidValue;
    p.heads_per_block = 16 / p.vall;
    if (p.heads_per_block > p.heads) p.heads_per_block = p.heads;
    p.nblk = (p.heads + p.heads_per_block - 1) / p.heads_per_block;
    const int64_t blocks = (int64_t)p.groups * p.n_tok * p.nblk;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(variate_attend, dim3((unsigned)blocks), dim3(64), 0, stream, p);
    return hipGetLastError();
}

}  // namespace tsfm
