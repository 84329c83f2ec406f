// KV cache for block-autoregressive decode (bf16 / f16, f32 accumulation) on gfx950.
//
// The reference has no cache: Timestral's blockDecode re-encodes the whole grown context every
// block (src/timestral/forecaster.zig:423-563), so the K/V of every unchanged prefix token is
// recomputed. With a causal encoder and a fixed prefix, rows [P, P + n) of causal selfAttend over
// the concatenated sequence equal n queries at positions P.. attending over cached keys, which is
// what tsfm_kv_attend computes.
//
// Layout (per (series, head), `cap` a multiple of 64 keys, set by tsfm_kv_create):
//   K: [cap][64] halves, one 128-byte row per key.
//   V: [cap/32][4][64][8] halves: 32-key chunks in the operand order of
//      v_mfma_f32_16x16x32_{bf16,f16} (see attn_half.hip): octet g of a chunk holds keys
//      {4g..4g+3, 16+4g..16+4g+3} of every dim, so a lane's A operand is one 16-byte load and a
//      16-lane group reads 256 contiguous bytes.
// Decode reads both straight from HBM with no LDS staging: one workgroup per
// (series, head, 32 queries); its four waves take 32-key tiles t = w, w+4, ... (fine enough that
// the waves of a 288..544-key decode block finish within a tile of each other) and merge their
// (max, sum, O) partials through LDS at the end (split-key flash decoding). The Q operands sit in
// LDS, read again every tile, so a wave holds 126 VGPRs and four workgroups (16 waves, 39 KB of
// LDS each) fit a CU: 1024 resident workgroups, each with the next tile's loads in flight.
#include "common.hpp"
#include "launch.hpp"

namespace tsfm {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int NK = 32;  // keys per tile: 16-key S blocks x NK / 16, 32-key V chunks x NK / 32
constexpr int NKB = NK / 16, NCH = NK / 32;
constexpr int NWAVE = 4;
constexpr int NT = 64 * NWAVE;
constexpr int QB = 32;  // queries per workgroup

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

// ---- append ----
// The 16-byte V slot that starts at key key0 (slot j holds key key0 + j for j < 4, key0 + 16 + (j - 4)
// for j >= 4) of one dim, after writing the new tokens [pos0, pos0 + n_new) into it; src points at
// that dim of new token 0. A slot the new tokens cover only in part is read first and its other
// keys kept.
__device__ __forceinline__ u32x4 v_slot(const u32x4* slot, const uint16_t* __restrict__ src, int64_t v_tok, int key0,
                                        int pos0, int n_new) {
    const bool whole = key0 >= pos0 && key0 + 19 < pos0 + n_new;  // uniform over the 64 dims
    u32x4 w = whole ? u32x4{0, 0, 0, 0} : *slot;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int t = key0 + (j < 4 ? j : 12 + j) - pos0;
        if (t < 0 || t >= n_new) continue;
        const uint32_t x = src[t * v_tok];
        w[j >> 1] = (j & 1) ? (w[j >> 1] & 0xffffu) | (x << 16) : (w[j >> 1] & 0xffff0000u) | x;
    }
    return w;
}

// K: one thread per (series, head, new token, 8-dim chunk): 16-byte load, 16-byte store.
// V: one thread per (series, head, touched 32-key chunk, octet, dim) builds the whole 16-byte slot
//    (8 keys of one dim) in registers and stores it once; consecutive threads take consecutive dims,
//    so the eight 2-byte loads (one per key, from eight token rows) and the store are all contiguous
//    across the wave. A slot the append covers only in part is read first and its other keys kept.
__global__ __launch_bounds__(256) void kv_append(KvLayout c, const uint16_t* __restrict__ k, int64_t k_tok,
                                                 int64_t k_batch, const uint16_t* __restrict__ v, int64_t v_tok,
                                                 int64_t v_batch, int32_t pos0, int32_t n_new, int64_t k_items,
                                                 int32_t ch0, int32_t nch) {
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id < k_items) {
        const int chunk = (int)(id & 7);
        int64_t rest = id >> 3;
        const int t = (int)(rest % n_new);
        rest /= n_new;
        const int h = (int)(rest % c.H);
        const int b = (int)(rest / c.H);
        const int64_t bh = (int64_t)b * c.H + h;
        const u32x4 kv = ldu4(k + b * k_batch + t * k_tok + h * kHeadDim + 8 * chunk);
        *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(c.k) + (bh * c.cap + pos0 + t) * kHeadDim + 8 * chunk) = kv;
        return;
    }
    const int64_t vid = id - k_items;
    if (vid >= (int64_t)c.B * c.H * nch * 4 * kHeadDim) return;
    const int d = (int)(vid & 63);
    const int o = (int)((vid >> 6) & 3);
    int64_t rest = vid >> 8;
    const int ch = ch0 + (int)(rest % nch);
    rest /= nch;
    const int h = (int)(rest % c.H);
    const int b = (int)(rest / c.H);
    const int64_t bh = (int64_t)b * c.H + h;
    u32x4* slot = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(c.v) +
                                           (((bh * (c.cap / 32) + ch) * 4 + o) * kHeadDim + d) * 8);
    *slot = v_slot(slot, v + b * v_batch + h * kHeadDim + d, v_tok, 32 * ch + 4 * o, pos0, n_new);
}

// ---- attend ----
// APPEND: the fused block decode of a 32-token block starting on a 32-key boundary (q_pos0 % 32 == 0,
// n_q == 32). The workgroup -- the only one that reads its (series, head) -- loads the block's K
// rows and its V chunk (built in the cache's slot order) once, writes them to the cache and to LDS,
// and the tile holding the new keys takes them from LDS. Only an LDS barrier separates the two:
// no wave waits for the cache writes, and each wave's first tile, if it holds old keys only, is
// loading meanwhile.
template <bool BF16, bool APPEND>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4, 4))) void kv_attend(
    KvLayout c, const uint16_t* __restrict__ q, int64_t q_tok, int64_t q_batch, uint16_t* __restrict__ o, int64_t o_tok,
    int64_t o_batch, int32_t n_q, int32_t q_pos0, int32_t n_k, float scale, KvNew nw) {
    // LDS: the Q operands, and the waves' partial results for the merge at the end or, with
    // APPEND, the block's new K rows and V chunk during the loop (the last two are separated by a
    // barrier and share their space).
    struct Merge {
        float m[NWAVE][QB], l[NWAVE][QB];
        float o[NWAVE][QB][kHeadDim + 4];
    };
    struct New {
        u32x4 k[QB * 8];          // [token][8 x 16 B]
        u32x4 v[4 * kHeadDim];    // [octet][dim] slots
    };
    constexpr size_t kLdsBytes = sizeof(Merge) > sizeof(New) ? sizeof(Merge) : sizeof(New);
    struct Qs {
        u32x4 f[2][2][64];  // the Q^T operands, [query block][dim half][lane]
    };
    __shared__ __attribute__((aligned(16))) char lds[sizeof(Qs) + kLdsBytes];
    Qs& qs = *reinterpret_cast<Qs*>(lds);
    Merge& mg = *reinterpret_cast<Merge*>(lds + sizeof(Qs));
    New& nwl = *reinterpret_cast<New*>(lds + sizeof(Qs));
    u32x4* const new_k = nwl.k;
    u32x4* const new_v = nwl.v;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ql = lane & 15, g = lane >> 4;
    const int qblocks = (n_q + QB - 1) / QB;
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = logical / qblocks, qbk = logical % qblocks;
    const int b = bh / c.H, h = bh % c.H;
    const int qi0 = qbk * QB;
    const int nqv = min(QB, n_q - qi0);           // valid queries of this workgroup
    const int qlo = q_pos0 + qi0;                  // position of its first query
    const int kend = min(n_k, qlo + nqv);          // keys any of its queries reads
    const int ntiles = (kend + NK - 1) / NK;
    const float c2 = scale * kLog2e;

    // Not __restrict__: with APPEND the kernel writes the new rows through Kw / Vw and reads them
    // back after the barrier.
    uint16_t* const Kw = static_cast<uint16_t*>(c.k) + (int64_t)bh * c.cap * kHeadDim;
    uint16_t* const Vw = static_cast<uint16_t*>(c.v) + (int64_t)bh * c.cap * kHeadDim;
    const uint16_t* const Kc = Kw;
    const uint16_t* const Vc = Vw;

    if (wave == 0) {
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            const int qi = qi0 + 16 * qb + ql;
            u32x4 lo = {0, 0, 0, 0}, hi = lo;
            if (qi < n_q) {
                const uint16_t* src = q + b * q_batch + (int64_t)qi * q_tok + h * kHeadDim + 8 * g;
                lo = ldu4(src);
                hi = ldu4(src + 32);
            }
            qs.f[qb][0][lane] = lo;
            qs.f[qb][1][lane] = hi;
        }
    }
    if (!APPEND) __syncthreads();

    float mc_run[2] = {kNegInf, kNegInf};
    float l_run[2] = {0.f, 0.f};
    f32x4 oacc[4][2];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int qb = 0; qb < 2; qb++) oacc[db][qb] = f32x4{0, 0, 0, 0};

    // Operand fragments of one tile, loaded straight from the cache. Rows past n_k (up to the
    // capacity) are read but always masked: the cache is zero-filled at creation, so they hold
    // finite values and contribute exactly 0.
    u32x4 kf[NKB][2], vf[NCH][4];
    // With APPEND, the 16-key blocks and the 32-key chunk of the new tokens come from LDS (the
    // choice is uniform: the new block is one whole chunk).
    auto load_k = [&](int kbase) {
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const int key0 = kbase + kb * 16;
            if (APPEND && key0 >= q_pos0 && key0 < q_pos0 + QB) {
                const u32x4* kr = new_k + (key0 - q_pos0 + ql) * 8 + g;
                kf[kb][0] = kr[0];
                kf[kb][1] = kr[4];
                continue;
            }
            const uint16_t* kr = Kc + (int64_t)(key0 + ql) * kHeadDim + 8 * g;
            kf[kb][0] = ldu4(kr);
            kf[kb][1] = ldu4(kr + 32);
        }
    };
    auto load_v = [&](int kbase) {
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            const int chunk = (kbase >> 5) + ch;
            if (APPEND && chunk == (q_pos0 >> 5)) {
#pragma unroll
                for (int db = 0; db < 4; db++) vf[ch][db] = new_v[g * kHeadDim + ql + 16 * db];
                continue;
            }
            const uint16_t* vr = Vc + (((int64_t)chunk * 4 + g) * kHeadDim + ql) * 8;
#pragma unroll
            for (int db = 0; db < 4; db++) vf[ch][db] = ldu4(vr + db * 16 * 8);
        }
    };

    int t = wave;
    if (APPEND) {
        // New K: one 16-byte piece per thread (32 tokens x 8). New V: one slot per thread (4 octets
        // x 64 dims of the block's chunk); slot j of octet oc holds token 4 oc + j (j < 4) or
        // 16 + 4 oc + (j - 4) of the block.
        const uint16_t* __restrict__ kn = static_cast<const uint16_t*>(nw.k) + b * nw.k_batch + h * kHeadDim;
        const uint16_t* __restrict__ vn = static_cast<const uint16_t*>(nw.v) + b * nw.v_batch + h * kHeadDim;
        const int tk = tid >> 3, pc = tid & 7, oc = tid >> 6, d = tid & 63;
        const u32x4 kin = ldu4(kn + (int64_t)tk * nw.k_tok + 8 * pc);
        u32x4 vin;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const int t0 = 4 * oc + (w < 2 ? 2 * w : 12 + 2 * w);  // tokens of halves 2w, 2w+1
            const uint32_t lo = vn[(int64_t)t0 * nw.v_tok + d], hi = vn[(int64_t)(t0 + 1) * nw.v_tok + d];
            vin[w] = lo | (hi << 16);
        }
        const bool early = t < ntiles && t * NK + NK <= q_pos0;  // the wave's first tile holds old keys only
        if (early) {
            load_k(t * NK);
            load_v(t * NK);
        }
        new_k[tid] = kin;
        new_v[tid] = vin;
        *reinterpret_cast<u32x4*>(Kw + (int64_t)(q_pos0 + tk) * kHeadDim + 8 * pc) = kin;
        *reinterpret_cast<u32x4*>(Vw + (((int64_t)(q_pos0 >> 5) * 4 + oc) * kHeadDim + d) * 8) = vin;
        // LDS only: the cache writes need not have landed (this workgroup reads the new rows from LDS).
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (!early && t < ntiles) {
            load_k(t * NK);
            load_v(t * NK);
        }
    } else if (t < ntiles) {
        load_k(t * NK);
        load_v(t * NK);
    }
    for (; t < ntiles; t += NWAVE) {
        const int kbase = t * NK;
        const int tn = t + NWAVE;
        asm volatile("" ::: "memory");  // Q is read from LDS every tile, not kept in registers
        u32x4 qf[2][2];
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            qf[qb][0] = qs.f[qb][0][lane];
            qf[qb][1] = qs.f[qb][1][lane];
        }
        f32x4 sacc[NKB][2];
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int qb = 0; qb < 2; qb++)
                sacc[kb][qb] = mfma<BF16>(kf[kb][1], qf[qb][1], mfma<BF16>(kf[kb][0], qf[qb][0], f32x4{0, 0, 0, 0}));
        if (tn < ntiles) load_k(tn * NK);

        const bool plain = kbase + NK - 1 <= qlo;  // every key of the tile is visible to every query
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            const int qpos = qlo + 16 * qb + ql;
            float mloc = kNegInf;
#pragma unroll
            for (int kb = 0; kb < NKB; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float x = sacc[kb][qb][r];
                    if (!plain && kbase + kb * 16 + 4 * g + r > qpos) x = kNegInf;
                    sacc[kb][qb][r] = x;
                    mloc = fmaxf(mloc, x);
                }
            const float mt = mloc == kNegInf ? kNegInf : mloc * c2;
            const float mn = fmaxf(max4(mt), mc_run[qb]);
            const float mc_use = mn == kNegInf ? 0.f : mn;
            const float alpha = __builtin_amdgcn_exp2f(mc_run[qb] - mc_use);
            mc_run[qb] = mn;
            float lsum = 0.f;
#pragma unroll
            for (int kb = 0; kb < NKB; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][qb][r], c2, -mc_use));
                    sacc[kb][qb][r] = e;
                    lsum += e;
                }
            l_run[qb] = l_run[qb] * alpha + lsum;
#pragma unroll
            for (int db = 0; db < 4; db++) oacc[db][qb] *= alpha;
        }

#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            u32x4 pf[2];
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                const f32x4 a = sacc[2 * ch][qb], d = sacc[2 * ch + 1][qb];
                pf[qb] = u32x4{pack2<BF16>(a[0], a[1]), pack2<BF16>(a[2], a[3]), pack2<BF16>(d[0], d[1]),
                               pack2<BF16>(d[2], d[3])};
            }
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int qb = 0; qb < 2; qb++) oacc[db][qb] = mfma<BF16>(vf[ch][db], pf[qb], oacc[db][qb]);
        }
        if (tn < ntiles) load_v(tn * NK);
    }

    // ---- merge the four waves' partial results ----
    if (APPEND) __syncthreads();  // every wave is done with the new rows in LDS
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const float l = sum4(l_run[qb]);
        const int qq = 16 * qb + ql;
        if (g == 0) {
            mg.m[wave][qq] = mc_run[qb];
            mg.l[wave][qq] = l;
        }
#pragma unroll
        for (int db = 0; db < 4; db++) st4(&mg.o[wave][qq][16 * db + 4 * g], oacc[db][qb]);
    }
    __syncthreads();
    {
        const int qq = tid >> 3, d0 = 8 * (tid & 7);  // 32 queries x 8 dim groups
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) M = fmaxf(M, mg.m[w][qq]);
        float L = 0.f;
        f32x4 a0 = {0, 0, 0, 0}, a1 = a0;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) {
            const float f = mg.m[w][qq] == kNegInf ? 0.f : __builtin_amdgcn_exp2f(mg.m[w][qq] - M);
            L += f * mg.l[w][qq];
            a0 += f * ld4(&mg.o[w][qq][d0]);
            a1 += f * ld4(&mg.o[w][qq][d0 + 4]);
        }
        if (qq < nqv) {
            const float inv = 1.0f / L;
            a0 *= inv;
            a1 *= inv;
            uint16_t* dst = o + b * o_batch + (int64_t)(qi0 + qq) * o_tok + h * kHeadDim + d0;
            *reinterpret_cast<u32x4*>(dst) = u32x4{pack2<BF16>(a0[0], a0[1]), pack2<BF16>(a0[2], a0[3]),
                                                   pack2<BF16>(a1[0], a1[1]), pack2<BF16>(a1[2], a1[3])};
        }
    }
}

}  // namespace

hipError_t launch_kv_append(const KvLayout& c, bool /*is_bf16*/, const void* k, int64_t k_tok, int64_t k_batch,
                            const void* v, int64_t v_tok, int64_t v_batch, int32_t pos0, int32_t n_new,
                            hipStream_t stream) {
    const int64_t k_items = (int64_t)c.B * c.H * n_new * 8;
    const int32_t ch0 = pos0 / 32, nch = (pos0 + n_new - 1) / 32 - ch0 + 1;
    const int64_t v_items = (int64_t)c.B * c.H * nch * 4 * kHeadDim;
    const int64_t blocks = (k_items + v_items + 255) / 256;
    if (n_new <= 0 || blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kv_append, dim3((unsigned)blocks), dim3(256), 0, stream, c,
                       static_cast<const uint16_t*>(k), k_tok, k_batch, static_cast<const uint16_t*>(v), v_tok,
                       v_batch, pos0, n_new, k_items, ch0, nch);
    return hipGetLastError();
}

hipError_t launch_kv_attend(const KvLayout& c, bool is_bf16, const void* q, int64_t q_tok, int64_t q_batch, void* o,
                            int64_t o_tok, int64_t o_batch, int32_t n_q, int32_t q_pos0, int32_t n_k, float scale,
                            hipStream_t stream) {
    const int64_t blocks = (int64_t)c.B * c.H * ((n_q + QB - 1) / QB);
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
    if (!(scale >= 0.f)) return hipErrorNotSupported;  // the row max is taken before scaling
    const KvNew none{};
    if (is_bf16)
        hipLaunchKernelGGL((kv_attend<true, false>), dim3((unsigned)blocks), dim3(NT), 0, stream, c,
                           static_cast<const uint16_t*>(q), q_tok, q_batch, static_cast<uint16_t*>(o), o_tok, o_batch,
                           n_q, q_pos0, n_k, scale, none);
    else
        hipLaunchKernelGGL((kv_attend<false, false>), dim3((unsigned)blocks), dim3(NT), 0, stream, c,
                           static_cast<const uint16_t*>(q), q_tok, q_batch, static_cast<uint16_t*>(o), o_tok, o_batch,
                           n_q, q_pos0, n_k, scale, none);
    return hipGetLastError();
}

hipError_t launch_kv_append_attend(const KvLayout& c, bool is_bf16, const KvNew& nw, const void* q, int64_t q_tok,
                                   int64_t q_batch, void* o, int64_t o_tok, int64_t o_batch, int32_t n_new,
                                   int32_t pos0, float scale, hipStream_t stream) {
    static_assert(kKvFusedBlock == QB, "one workgroup per (series, head)");
    const int64_t blocks = (int64_t)c.B * c.H;
    if (n_new != QB || pos0 < 0 || pos0 % 32 != 0 || pos0 + n_new > c.cap || blocks <= 0 || blocks > 0x7fffffff)
        return hipErrorInvalidValue;
    if (!(scale >= 0.f)) return hipErrorNotSupported;  // the row max is taken before scaling
    if (is_bf16)
        hipLaunchKernelGGL((kv_attend<true, true>), dim3((unsigned)blocks), dim3(NT), 0, stream, c,
                           static_cast<const uint16_t*>(q), q_tok, q_batch, static_cast<uint16_t*>(o), o_tok, o_batch,
                           n_new, pos0, pos0 + n_new, scale, nw);
    else
        hipLaunchKernelGGL((kv_attend<false, true>), dim3((unsigned)blocks), dim3(NT), 0, stream, c,
                           static_cast<const uint16_t*>(q), q_tok, q_batch, static_cast<uint16_t*>(o), o_tok, o_batch,
                           n_new, pos0, pos0 + n_new, scale, nw);
    return hipGetLastError();
}

}  // namespace tsfm
