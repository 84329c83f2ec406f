// Host-side launchers of the device kernels. Each returns the launch's hipError_t.
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace tsfm {

// f32 q/k/v/o; mask = TSFM_MASK_*, bias = BiasKind.
hipError_t launch_attn_f32(const Params& p, int mask, int bias, bool rope, hipStream_t stream);

// bf16 (is_bf16) or f16 q/k/v/o, f32 accumulation.
hipError_t launch_attn_half(const Params& p, bool is_bf16, int mask, int bias, bool rope, hipStream_t stream);

// KV cache: device layout and kernels (kv_cache.hip).
struct KvLayout {
    void* k;          // [B][H][cap][64]
    void* v;          // [B][H][cap/32][4][64][8]  (32-key chunks, matrix-core operand order)
    int32_t B, H, cap;  // cap: a multiple of 64
};
hipError_t launch_kv_append(const KvLayout& c, bool is_bf16, const void* k, int64_t k_tok, int64_t k_batch,
                            const void* v, int64_t v_tok, int64_t v_batch, int32_t pos0, int32_t n_new,
                            hipStream_t stream);
hipError_t launch_kv_attend(const KvLayout& c, bool is_bf16, const void* q, int64_t q_tok, int64_t q_batch,
                            void* o, int64_t o_tok, int64_t o_batch, int32_t n_q, int32_t q_pos0, int32_t n_k,
                            float scale, hipStream_t stream);

}  // namespace tsfm
