/*
 * tsfm_attn.h -- C ABI of libtsfm_attn.so, the gfx950 (MI355X) attention path for tsfm-zig.
 *
 * Drop-in boundary. In the reference every attention call funnels through
 *   core.attn.selfAttend / selfAttendRuntime        src/core/attn.zig:72-117
 * called once per (series, head) from a fork-join job:
 *   Chronos-Bolt encoder   par.forRange(nb*nh, SelfJob.attend)   src/chronos_bolt/model.zig:243, 317-346
 *   Chronos-Bolt decoder   par.forRange(nb*nh, CrossJob.attend)  src/chronos_bolt/model.zig:297, 349-381
 *   Chronos-2 time attn    RoPE loop + forRange(b*nh, TimeJob)   src/chronos2/model.zig:236-245, 260, 277-309
 *   Timestral time attn    forRange(rows*nh, TimeJob.attend)     src/timestral/model.zig:513-515, 558-635
 * and its arithmetic reaches a device only as two GEMMs per (series, head) through
 *   Backend.sgemmNT / sgemmNN                        src/platform/backend.zig:51-57
 *   cuda_sgemm_nt / cuda_sgemm_nn                    src/platform/cuda/gemm.c:316-330
 * tsfm_attn_fwd() replaces one whole forRange(B*H, Job.attend) call: the caller keeps its Zig
 * signatures and, at the forRange call site, tries one batched call first and runs its unchanged
 * per-item CPU loop when the call returns non-zero.
 *
 * Conventions (the reference backend's, src/platform/cuda/gemm.c:1-16, backend.zig:33-36):
 *   - every entry point returns 0 on success; any other value means "not run, use the CPU path"
 *     and promises no partial output. Nothing here aborts the process;
 *   - the caller owns every buffer it passes; the library never frees caller memory;
 *   - the library is thread-safe: device set-up runs once (pthread_once), and each host thread
 *     gets its own HIP stream and device staging buffers, released when the thread exits; the
 *     device-pointer model calls keep their scratch per (thread, stream, entry point) between
 *     calls, released the same way;
 *   - results do not depend on how many host threads call in, nor on batch composition: there
 *     are no atomics in any reduction and tile order is fixed.
 *
 * Layouts follow the reference: element (b, t, h, c) of Q lives at
 *   q[b * q_batch + t * q_tok + h * head_dim + c]
 * (`attn.Strides`, src/core/attn.zig:32, plus a batch stride). The supported head_dim is 64.
 */
#ifndef TSFM_ATTN_H
#define TSFM_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSFM_ATTN_ABI_VERSION 1

/* Return codes. Non-zero always means "fall back to the CPU". */
enum {
    TSFM_OK = 0,
    TSFM_E_UNAVAILABLE = 1, /* no gfx950 device / HIP runtime, or TSFM_HIP_DISABLE is set */
    TSFM_E_UNSUPPORTED = 2, /* valid request this library does not implement (shape, dtype, stride) */
    TSFM_E_INVALID = 3,     /* malformed arguments */
    TSFM_E_DEVICE = 4       /* a HIP call failed */
};

/* Mask variants. Values 0..4 are `attn.Mask` in declaration order (src/core/attn.zig:10-21):
 *   FULL           every query reads every key
 *   KEYS_ADDITIVE  invalid keys get -FLT_MAX added to their score (T5)
 *   CAUSAL         query i reads keys 0..=i
 *   CAUSAL_KEYS    causal over valid keys, diagonal always open (-inf elsewhere)
 *   FULL_KEYS      bidirectional over valid keys, diagonal always open
 * DECODER is the Timestral decoder-row mask written inline in TimeJob.attend
 * (src/timestral/model.zig:612-632): query i reads valid keys in [0, ctx_keys) and the chain
 * [chain_start, q_pos0 + i]; everything else gets -inf.
 * For masks 2..5, query i sits at key index q_pos0 + i ("i" and "j == i" in attn.zig). */
enum {
    TSFM_MASK_FULL = 0,
    TSFM_MASK_KEYS_ADDITIVE = 1,
    TSFM_MASK_CAUSAL = 2,
    TSFM_MASK_CAUSAL_KEYS = 3,
    TSFM_MASK_FULL_KEYS = 4,
    TSFM_MASK_DECODER = 5
};

/* Element type of q, k, v and o. Reference arithmetic is f32 (half checkpoints are widened at load,
 * src/core/safetensors.zig:81-91); BF16/F16 are new here and accumulate in f32. */
enum { TSFM_DTYPE_F32 = 0, TSFM_DTYPE_BF16 = 1, TSFM_DTYPE_F16 = 2 };

/* flags */
#define TSFM_ATTN_DEVICE_PTRS 1u /* every pointer is device memory; the call is asynchronous on `stream` */
#define TSFM_TIMESTRAL_BF16_ATTN 2u /* tsfm_timestral_forecast: time attention in bf16 (see there) */
/* The forecast entry points (tsfm_bolt_forecast, tsfm_bolt_forecast_horizon, tsfm_chronos2_forecast,
 * tsfm_timestral_forecast), together with TSFM_ATTN_DEVICE_PTRS: the per-call arrays (inputs,
 * observed, covariates, out) are host memory, the weights and every other model pointer device
 * memory (a host caller makes them once with tsfm_weight_register). The call copies the arrays in,
 * runs on the calling thread's own stream (the `stream` fields are not read), copies out back and
 * returns when it is written. */
#define TSFM_FORECAST_HOST_IO 4u

/* One batched attention call: o = softmax(mask(scale * q k^T + bias)) v for every (b, h).
 * Replaces: selfAttendRuntime per item (src/core/attn.zig:99-117) inside the forRange calls listed
 * above; the Chronos-2 serial RoPE loop (src/chronos2/model.zig:236-245) when rope_cos is set; the
 * positionBias materialisation (src/chronos_bolt/model.zig:195-205) when rel_table is set. */
typedef struct tsfm_attn_args {
    int32_t dtype;       /* TSFM_DTYPE_* */
    int32_t mask;        /* TSFM_MASK_* */
    int32_t batch;       /* B: series (Bolt, Chronos-2) or rows (Timestral) */
    int32_t heads;       /* H */
    int32_t n_q;         /* queries per (b, h) */
    int32_t n_k;         /* keys per (b, h) */
    int32_t head_dim;    /* D; 64 */
    int32_t q_pos0;      /* key index of query 0 (masks 2..5 and the RoPE position of queries) */
    int32_t ctx_keys;    /* DECODER: context keys are [0, ctx_keys) */
    int32_t chain_start; /* DECODER: first key of the decoder chain */
    float scale;         /* score scale (attn.selfAttend `scale`) */
    uint32_t flags;      /* TSFM_ATTN_DEVICE_PTRS or 0 (host pointers, synchronous) */

    const void *q;  int64_t q_tok, q_batch; /* element strides */
    const void *k;  int64_t k_tok, k_batch;
    const void *v;  int64_t v_tok, v_batch;
    void *o;        int64_t o_tok, o_batch;

    /* One byte per key, non-zero = valid (Zig `[]const bool`), row b at key_valid + b * kv_batch.
     * Read by masks KEYS_ADDITIVE, CAUSAL_KEYS, FULL_KEYS (n_k bytes per row) and DECODER
     * (min(n_k, ctx_keys) bytes per row); may be NULL for the others. */
    const uint8_t *key_valid; int64_t kv_batch;

    /* Additive score bias, applied before the mask (src/core/attn.zig:93). At most one of:
     *  - dense: bias[h * bias_head + i * bias_row + j], shared by every b (positionBias layout);
     *  - T5 relative: bias = rel_table[rel_bucket[j - i + n_q - 1] * heads + h], where rel_table is
     *    the (rel_buckets, heads) table (src/chronos_bolt/model.zig:115) and rel_bucket holds
     *    n_q + n_k - 1 bucket ids (tsfm_t5_bucket_table). Requires q_pos0 == 0. */
    const float *bias; int64_t bias_head, bias_row;
    const float *rel_table; const int32_t *rel_bucket; int32_t rel_buckets;

    /* Rotate-half RoPE applied to q and k before the product (nn.ropeHalf, src/core/nn.zig:448-467),
     * NULL rope_cos = none. Tables are (positions, rope_half) f32; key j uses row j, query i row
     * q_pos0 + i, of table number t = (rope_row0 + b) / rope_rows_per_table, which starts at
     * t * rope_table_stride. rope_half must be head_dim / 2. rope_rows_per_table = 0 means one
     * table shared by every b (Chronos-2); Timestral has one table per series group of
     * rope_rows_per_table rows, and rope_row0 is the group position of batch row 0. */
    const float *rope_cos, *rope_sin;
    int32_t rope_half; int32_t rope_rows_per_table; int32_t rope_row0; int64_t rope_table_stride;

    void *stream; /* hipStream_t the call is queued on with TSFM_ATTN_DEVICE_PTRS (NULL = the null
                   * stream, as in every HIP call); host-pointer calls use the thread's own stream */
} tsfm_attn_args;

/* Device set-up, run once per process (cuda/gemm.c:112-166 init_cuda / ensure_cuda). Optional:
 * every entry point calls it. Returns TSFM_OK or TSFM_E_UNAVAILABLE. */
int tsfm_attn_init(void);

/* 1 when the library can run (gfx950 device present, not disabled), else 0.
 * Counterpart of gpu.context() returning a backend or null (src/platform/cuda/gpu.zig:95-97). */
int tsfm_attn_available(void);

/* Batched attention (see tsfm_attn_args). */
int tsfm_attn_fwd(const tsfm_attn_args *args);

/* Human-readable reason for this thread's last non-zero return ("" if none). */
const char *tsfm_attn_last_error(void);

/* T5 bidirectional relative-position bucket of rel = key - query, with the reference's float32
 * log (src/chronos_bolt/model.zig:74-85). Host function. */
uint32_t tsfm_t5_relative_bucket(int64_t rel, uint32_t num_buckets, uint32_t max_distance);

/* Fills out[t] = tsfm_t5_relative_bucket(t - (n_q - 1), ...) for t in [0, n_q + n_k - 1): the
 * rel_bucket array of tsfm_attn_args. Host function; the bucket half of positionBias
 * (src/chronos_bolt/model.zig:195-205). Returns TSFM_OK or TSFM_E_INVALID. */
int tsfm_t5_bucket_table(int32_t *out, int32_t n_q, int32_t n_k, uint32_t num_buckets, uint32_t max_distance);

/* ---------------------------------------------------------------------------------------------
 * Timestral variate attention. Replaces the forRangeMin(groups * sl, VariateJob.run) call of
 * Model.variateAttention (src/timestral/model.zig:525-544, job at :648-709) and, when gate is set,
 * the nn.mulSigmoid that follows it (:541, src/core/nn.zig:423-433).
 *
 * At every (series group g, token slot t) the vall rows r = g * vall + i of the group attend each
 * other, per head: o[r, t, h] = sum_j softmax_j(scale * q[r, t, h] . k[g*vall + j, t, h]) v[...].
 * Row i may read row j when i == j, or when (t >= n_enc or key_valid[(g*vall + j) * kv_row + t])
 * and, with cov != 0, neither (role[i] != TARGET and role[j] == TARGET) nor (role[i] == KNOWN and
 * role[j] != KNOWN). Roles are model.Role in declaration order (src/timestral/model.zig:89).
 * With gate != NULL the result is multiplied by sigmoid(gate) (same layout as o) before it is stored.
 * f32 only; vall <= TSFM_VARIATE_MAX_ROWS (more rows: TSFM_E_UNSUPPORTED, use the CPU path);
 * head_dim 64. */
enum { TSFM_ROLE_TARGET = 0, TSFM_ROLE_PAST = 1, TSFM_ROLE_KNOWN = 2 };
#define TSFM_VARIATE_MAX_ROWS 256

typedef struct tsfm_variate_args {
    int32_t dtype;     /* TSFM_DTYPE_F32 */
    int32_t groups;    /* series */
    int32_t vall;      /* rows per series, 1..TSFM_VARIATE_MAX_ROWS */
    int32_t n_tok;     /* token slots per row (sl = ne + h) */
    int32_t n_enc;     /* encoder slots (ne): key_valid applies to slots t < n_enc */
    int32_t heads;     /* H; d_model = heads * head_dim */
    int32_t head_dim;  /* 64 */
    int32_t cov;       /* non-zero: the covariate firewalls apply */
    float scale;       /* 1/sqrt(head_dim) in the reference */
    uint32_t flags;    /* TSFM_ATTN_DEVICE_PTRS or 0 */
    /* Fused projection, element (r, t, part, h, c) at qkv + r*qkv_row + t*qkv_tok + part*heads*64
     * + h*64 + c with part 0/1/2 = q/k/v (the permuted (token, qkv, head, head_dim) layout,
     * src/timestral/model.zig:72-85). */
    const void *qkv; int64_t qkv_row, qkv_tok;
    void *o;         int64_t o_row, o_tok;     /* (r, t, h, c) */
    const void *gate; int64_t gate_row, gate_tok; /* optional, as o */
    const uint8_t *key_valid; int64_t kv_row;   /* (rows, n_enc) bytes */
    const uint8_t *roles;                       /* vall bytes of host memory: role of row i of every
                                                   series (read at the call; may be NULL when cov = 0) */
    void *stream;
} tsfm_variate_args;

int tsfm_variate_attend(const tsfm_variate_args *args);

/* ---------------------------------------------------------------------------------------------
 * Fused projection ahead of time attention, with RoPE in its epilogue. Replaces, in one launch:
 *  - Chronos-2: nn.linear for q, k and v and the serial RoPE loop (src/chronos2/model.zig:232-245);
 *  - Timestral: the fused qkv nn.linear over the permuted weight, the gate nn.linear and
 *    TimeJob.rope (src/timestral/model.zig:495,500,513,558-577): pass w_q/w_k/w_v = the three
 *    (d, d) blocks of the permuted weight and q/k/v = qkv, qkv + d, qkv + 2d with stride 3d;
 *  - Timestral variate attention: the same projections without RoPE (:532,535);
 *  - Chronos-Bolt: the q, k, v nn.linear calls of the encoder self-attention, no RoPE
 *    (src/chronos_bolt/model.zig:239-241).
 * For every token r = b * seq + t (r < batch * seq) of x (element (r, c) at x[r * x_tok + c]):
 *   q[r * q_tok + n] = (x[r, :] . w_q[n, :]) for n < heads * head_dim, then nn.ropeHalf on each
 *   head of q and k when rope_cos is set (token t of series row b uses row t of table
 *   (rope_row0 + b) / rope_rows_per_table, as in tsfm_attn_args); v and gate likewise, no RoPE.
 * Weights are nn.Weight's (out, in) row-major f32 (src/core/nn.zig:270-293, no bias). f32 only;
 * head_dim 64; d_in a multiple of 16; strides in elements, multiples of 4. */
typedef struct tsfm_proj_args {
    int32_t dtype;      /* TSFM_DTYPE_F32 */
    int32_t batch;      /* series (rows) */
    int32_t seq;        /* tokens per series */
    int32_t d_in;       /* width of x (d_model); a multiple of 16 */
    int32_t heads;      /* each output has heads * head_dim columns */
    int32_t head_dim;   /* 64 */
    uint32_t flags;     /* TSFM_ATTN_DEVICE_PTRS or 0 */
    int32_t rope_half;  /* 32 when rope_cos is set */
    int32_t rope_rows_per_table, rope_row0;
    int32_t out_dtype;  /* element type of q/k/v/gate: TSFM_DTYPE_F32, _BF16 or _F16 (rounded once,
                         * to nearest even, from the f32 result; feeds the half-precision attention) */
    int64_t rope_table_stride;
    const float *x; int64_t x_tok;
    const float *w_q, *w_k, *w_v;
    const float *w_gate;            /* optional; with gate */
    void *q;    int64_t q_tok;      /* strides in elements of out_dtype */
    void *k;    int64_t k_tok;
    void *v;    int64_t v_tok;
    void *gate; int64_t gate_tok;   /* optional; with w_gate */
    const float *rope_cos, *rope_sin;
    void *stream;
} tsfm_proj_args;

int tsfm_qkv_project(const tsfm_proj_args *args);

/* tsfm_qkv_project that allocates nothing. No counterpart in the reference: it is for callers that
 * cannot allocate device memory while they run (code under HIP graph capture, serving loops that
 * forbid hipMalloc). Same arguments and the same result bits as tsfm_qkv_project; device pointers
 * only (TSFM_ATTN_DEVICE_PTRS; host pointers return TSFM_E_UNSUPPORTED), queued on args->stream.
 * Small products split their reduction over workgroups; their partial sums go to one 16 MiB array
 * in the library's device memory per GPU, shared by every call on that GPU and kept between
 * calls: calls that overlap on one GPU (other streams or threads) race and must be serialised by
 * the caller. The split rule keeps every product's partials within the array (at most two splits
 * of 511 tiles of 64 x 64 floats: 16744448 bytes); a product that needed more would return
 * TSFM_E_UNSUPPORTED. */
int tsfm_qkv_project_noalloc(const tsfm_proj_args *args);

/* ---------------------------------------------------------------------------------------------
 * Chronos-2 encoder stack: Model.encode's layer loop and final norm (src/chronos2/model.zig:144-206)
 * in one call, every product on the matrix cores. Per layer, on x (batch * seq tokens of d_model):
 *   x += o(attn(rope(q(n1(x))), rope(k(n1(x))), v(n1(x))))   time attention (:208-262), the mask
 *        Mask.pick(false, keys_all_valid, true), the given scale (the model passes 1.0, :306);
 *   x += o_g(v_g(n2(x)))                                       group attention, singleton groups (:264-269);
 *   x += wo(relu(wi(n3(x))))                                   the MLP (:198-202);
 * with n1..n3 the layer's rmsNorms (nn.rmsNorm, src/core/nn.zig:361-396), then x = rmsNorm(x, final_norm).
 * x is the embedded tokens in and the hidden states out. Weights are nn.Weight's (out, in)
 * row-major f32. head_dim 64, d_model = heads * 64, d_ff a multiple of 16. With
 * TSFM_ATTN_DEVICE_PTRS every pointer (x, key_valid, tables, weights, final_norm; not `layers`
 * itself) is device memory and the call is asynchronous on `stream` (its scratch is allocated
 * and freed in stream order); with host pointers it uploads everything and returns when x is
 * written back. */
typedef struct tsfm_chronos2_layer {
    const float *time_norm;                          /* (d) */
    const float *time_q, *time_k, *time_v, *time_o;  /* (d, d) */
    const float *group_norm;                         /* (d) */
    const float *group_v, *group_o;                  /* (d, d) */
    const float *mlp_norm;                           /* (d) */
    const float *mlp_wi;                             /* (d_ff, d) */
    const float *mlp_wo;                             /* (d, d_ff) */
} tsfm_chronos2_layer;

typedef struct tsfm_chronos2_encode_args {
    int32_t batch;           /* series b */
    int32_t seq;             /* tokens per series (n_ctx + 1 + n_out) */
    int32_t d_model, heads, head_dim, d_ff, n_layers;
    int32_t keys_all_valid;  /* non-zero: every key_valid byte is set (Mask.pick -> FULL) */
    float eps;               /* layer_norm_epsilon */
    float scale;             /* time-attention score scale */
    uint32_t flags;          /* TSFM_ATTN_DEVICE_PTRS or 0 */
    float *x;                /* (b * seq, d_model), in place */
    const uint8_t *key_valid;          /* (b, seq) */
    const float *rope_cos, *rope_sin;  /* (seq, head_dim / 2) */
    const tsfm_chronos2_layer *layers; /* n_layers entries, host memory */
    const float *final_norm;           /* (d) */
    void *stream;
} tsfm_chronos2_encode_args;

int tsfm_chronos2_encode(const tsfm_chronos2_encode_args *args);

/* ---------------------------------------------------------------------------------------------
 * Chronos-2 model forward: the model part of the forecaster's runChunk
 * (src/chronos2/forecaster.zig:155-183) in one call:
 *   the input embedding (ResBlock, src/core/resblock.zig:63-79) of the context and future patch
 *   features -> the sequence [context; REG; future] with its key_valid (:162-173) -> the encoder
 *   stack (tsfm_chronos2_encode) -> the future tokens' hidden states (:177-181) -> the output head
 *   (ResBlock) -> raw (batch * n_out, num_quantiles * patch), before the forecaster's inverse
 *   scaling. The instance norm, patch features and inverse scaling (:88-153, :184-201) are per-series
 *   scalar loops and stay with the caller. */
typedef struct tsfm_resblock {
    const float *hidden_w, *hidden_b;      /* (hid, in), (hid) */
    const float *output_w, *output_b;      /* (out, hid), (out) */
    const float *residual_w, *residual_b;  /* (out, in), (out) */
    int32_t in, hid, out;                  /* in, hid multiples of 16; out of 4 */
    int32_t act;                           /* 0 = ReLU (ResBlock(.relu), Chronos), 1 = SiLU (ResBlock(.silu),
                                            * Timestral); biases may be NULL where the model has none */
} tsfm_resblock;

typedef struct tsfm_chronos2_forward_args {
    tsfm_chronos2_encode_args enc;  /* model dims, layers, final_norm, tables, eps, scale, flags, stream,
                                     * keys_all_valid (of the context patches); enc.seq = n_ctx + 1 + n_out;
                                     * enc.x and enc.key_valid are not read */
    int32_t n_ctx, n_out;           /* context and future patches per series */
    const float *feats;             /* (batch * n_ctx, 3 * patch) [time_enc, values, mask] features */
    const float *fut_feats;         /* (batch * n_out, 3 * patch) */
    const uint8_t *ctx_valid;       /* (batch, n_ctx): the patch has an observation */
    const float *reg;               /* (d_model) the [REG] token */
    tsfm_resblock input_embed, output_embed;
    float *raw;                     /* (batch * n_out, output_embed.out) */
} tsfm_chronos2_forward_args;

int tsfm_chronos2_forward(const tsfm_chronos2_forward_args *args);

/* The whole Chronos-2 forecast of a block of series (runChunk, src/chronos2/forecaster.zig:59-204)
 * on device memory: per series the instance norm over the observed values (NaN = missing; a
 * zero scale becomes 1e-5), the [time_enc, values, mask] features of the context patches
 * (left-padded to whole patches, values optionally asinh'd) and of the future patches, the model
 * forward, and the inverse scaling into out (batch, horizon, q) in the model's quantile order.
 * Row s of the inputs is inputs[s * stride + start ..][0..len] (forecast() passes stride = t_in
 * and start = t_in - len after truncating to context_length, :27-36). patch = input_embed.in / 3;
 * q = output_embed.out / patch; model.n_ctx must be ceil(len / patch) and model.n_out
 * ceil(horizon / patch). model.feats, fut_feats, ctx_valid, raw and enc.keys_all_valid are not read
 * (the additive key mask is used). Device weights (TSFM_ATTN_DEVICE_PTRS in model.enc.flags); inputs
 * and out are device memory too, or host memory with TSFM_FORECAST_HOST_IO (synchronous). */
typedef struct tsfm_chronos2_forecast_args {
    tsfm_chronos2_forward_args model;
    const float *inputs; int64_t stride, start;
    int32_t len;        /* context steps per series */
    int32_t horizon;    /* forecast steps, 1 .. n_out * patch */
    float time_scale;   /* chronos_config.time_encoding_scale */
    int32_t arcsinh;    /* chronos_config.use_arcsinh */
    float *out;         /* (batch, horizon, q) */
} tsfm_chronos2_forecast_args;

int tsfm_chronos2_forecast(const tsfm_chronos2_forecast_args *args);

/* ---------------------------------------------------------------------------------------------
 * Chronos-Bolt model forward: the model part of the forecaster's chunk
 * (src/chronos_bolt/forecaster.zig:199-213) in one call:
 *   input embedding (ResBlock(.relu)) of the [values, mask] patch features -> [patches; REG] with
 *   its key validity -> the T5 encoder (Model.encode, src/chronos_bolt/model.zig:210-254: rmsNorm,
 *   q/k/v, self-attention with the T5 relative bias and the additive key mask at scale 1, o, ReLU FFN,
 *   each added back; final norm) -> the one-token decoder (Model.decode, :258-308: self-attention
 *   over one token = o(v(x)), cross-attention to the encoder output, ReLU FFN; final norm) -> the
 *   output head (ResBlock) -> raw (batch, output_embed.out), before the inverse instance norm.
 * The T5 bucket ids are computed on the host with the reference's float32 formula
 * (tsfm_t5_bucket_table). Requires use_reg (Chronos-Bolt checkpoints set use_reg_token). */
typedef struct tsfm_bolt_enc_layer {
    const float *attn_norm, *q, *k, *v, *o;   /* norm (d); q/k/v (inner, d); o (d, inner) */
    const float *ffn_norm, *wi, *wo;          /* norm (d); wi (d_ff, d); wo (d, d_ff) */
} tsfm_bolt_enc_layer;

typedef struct tsfm_bolt_dec_layer {
    const float *self_norm, *self_v, *self_o;                           /* (d); (inner, d); (d, inner) */
    const float *cross_norm, *cross_q, *cross_k, *cross_v, *cross_o;  /* (d); (inner, d) x3; (d, inner) */
    const float *ffn_norm, *wi, *wo;
} tsfm_bolt_dec_layer;

typedef struct tsfm_bolt_forward_args {
    int32_t batch, n_patch;          /* series; context patches (seq = n_patch + 1 with [REG]) */
    int32_t d_model, heads, head_dim, d_ff;  /* head_dim = d_kv = 64; inner = heads * head_dim */
    int32_t n_enc_layers, n_dec_layers;
    int32_t keys_all_valid;          /* every patch observed (Mask.pick -> FULL) */
    int32_t rel_buckets, rel_max_distance;
    float eps;
    uint32_t flags;                  /* TSFM_ATTN_DEVICE_PTRS or 0 */
    const float *feats;              /* (batch * n_patch, input_embed.in) [values, mask] */
    const uint8_t *patch_valid;      /* (batch, n_patch) */
    const float *reg;                /* (d) the [REG] embedding */
    const float *dec_start;          /* (d) the decoder start token embedding */
    const float *rel_table;          /* (rel_buckets, heads), shared by every encoder layer */
    const tsfm_bolt_enc_layer *enc_layers;  /* host memory */
    const float *enc_final_norm;
    const tsfm_bolt_dec_layer *dec_layers;  /* host memory */
    const float *dec_final_norm;
    tsfm_resblock input_embed, output_embed;
    float *raw;                      /* (batch, output_embed.out) */
    void *stream;
} tsfm_bolt_forward_args;

int tsfm_bolt_forward(const tsfm_bolt_forward_args *args);

/* The whole Chronos-Bolt forecast of a block of series (predictBlock/runChunk,
 * src/chronos_bolt/forecaster.zig:115-220) on device memory: per series the instance norm over the
 * observed values (NaN = missing) and the [values, mask] patch features left-padded to whole
 * patches, the model forward, and the inverse norm. Row s of the context is
 * ctx[s * stride + offset ..][0..len]; out is (batch, q * P) = (batch, output_embed.out).
 * model.n_patch must be ceil(len / patch); model.feats, model.patch_valid, model.raw and
 * model.keys_all_valid are not read (the additive key mask is used: the same weights as FULL when
 * every patch is observed). Device weights (TSFM_ATTN_DEVICE_PTRS in model.flags); ctx and out are
 * device memory too, or host memory with TSFM_FORECAST_HOST_IO in model.flags (synchronous). */
typedef struct tsfm_bolt_forecast_args {
    tsfm_bolt_forward_args model;
    const float *ctx; int64_t stride, offset;
    int32_t len;        /* context steps per series */
    int32_t patch;      /* input_patch_size; input_embed.in = 2 * patch */
    float norm_eps;     /* the scale of a series with zero spread (forecaster.zig:18: 1e-5) */
    float *out;
} tsfm_bolt_forecast_args;

int tsfm_bolt_forecast(const tsfm_bolt_forecast_args *args);

/* Chronos-Bolt forecaster.forecast (src/chronos_bolt/forecaster.zig:22-78) on device memory: any
 * horizon. The first block forecasts prediction_length steps from the last context_length steps of
 * each series; while the horizon is not reached, every quantile path becomes its own context row
 * (the window grows by prediction_length steps, its oldest steps dropped past context_length), the
 * q x q rows of a series give q * q samples per step, and the next block is their empirical
 * quantiles at quantile_levels (torch.quantile's linear interpolation, quantileLinear :81-92).
 * model: the weights and dims (batch = series); model.n_patch, feats, patch_valid, raw and
 * keys_all_valid are not read. inputs (batch, t_in) f32, NaN = missing; out (batch, horizon, q).
 * Device weights; inputs and out device memory (asynchronous on model.stream) or, with
 * TSFM_FORECAST_HOST_IO in model.flags, host memory (synchronous). */
typedef struct tsfm_bolt_horizon_args {
    tsfm_bolt_forward_args model;
    const float *inputs;
    int32_t t_in, horizon;
    int32_t patch;              /* input_patch_size; input_embed.in = 2 * patch */
    int32_t prediction_length;  /* P: output_embed.out = n_quantiles * P */
    int32_t context_length;     /* the window of every block */
    int32_t n_quantiles;        /* 1..16 */
    const float *quantile_levels;  /* host, n_quantiles (the config's quantiles as f32) */
    float norm_eps;
    float *out;
} tsfm_bolt_horizon_args;

int tsfm_bolt_forecast_horizon(const tsfm_bolt_horizon_args *args);

/* ---------------------------------------------------------------------------------------------
 * Timestral forecast: forecaster.forecast (src/timestral/forecaster.zig:57-180) of a batch of
 * series of target variates, optionally with numeric past-only and known-future covariate rows
 * (Covariates.past / .known, :36-46), f32: device weights, and inputs, observed, covariates and
 * out in device memory (asynchronous on `stream`) or, with TSFM_FORECAST_HOST_IO, host memory.
 * Categorical covariates (Covariates.cat_past / .cat_known) are target-encoded into numeric rows
 * by the caller first (tsfm_timestral_encode_categorical below) and passed as past / known rows.
 * The whole forecast runs on the device: forecastRaw's forward-fill and left padding (:303-394),
 * the decode loop of blockDecode (:423-563) with predictBlock (src/timestral/model.zig:220-432:
 * causal per-patch statistics, patch embedding, the time / variate transformer, the monotone
 * quantile head) and refineBlock (:582-662), the median feedback and max_context window, the
 * quantile cap (:396-418), the mirrored pass of the symmetric average (:107-137, run in the same
 * batch) and the non-negative clip (:163-178). A forecast whose output contains NaN is returned as
 * is (the reference reports error.DegenerateInput).
 * With kv_cache set and no known-future covariates, decode blocks after the first run only their
 * new patches and decoder tokens, attending over the time-attention K/V the earlier blocks
 * computed (the reference re-encodes the whole context every block; the result is the same
 * computation, up to f32 summation order); blocks after a max_context drop re-encode in full.
 * Past-only covariate rows keep that: every row's encoder tokens are then causal in time (causal
 * per-patch statistics, causal time attention, variate attention within a token slot), and the
 * window's blank future patches, which no context token or decoder query reads, are recomputed as
 * context in the next block. Known-future rows attend over the whole window and take whole-window
 * statistics, so every token changes when the window grows: with them kv_cache is ignored and
 * every block re-encodes.
 * With TSFM_TIMESTRAL_BF16_ATTN in flags the time attention runs on the bf16 matrix cores: the q/k/v
 * projections are rounded once to bf16 (after RoPE) into a bf16 K/V cache, the attention keeps f32
 * scores, softmax and accumulation, and its output is rounded to bf16 and widened back to f32 for
 * the gate and the out projection. Everything else stays f32. The reference has no such mode (its
 * time attention is f32); a bf16 forecast agrees with the f32 one to about 1e-2 of the forecast's
 * scale when the model works in linear space. With use_asinh the head's outputs are sinh-expanded,
 * which turns bf16's relative rounding into a relative error of the forecast several times larger:
 * that combination returns TSFM_E_UNSUPPORTED.
 * Errors as the reference's: covariates with covariate_enabled == 0 (error.CovariatesUnsupported),
 * known covariates with a schedule that cannot route them (error.KnownCovariatesUnsupported) return
 * TSFM_E_UNSUPPORTED; a covariate array with a zero count, or a count without its array, returns
 * TSFM_E_INVALID (error.InvalidInput). */
typedef struct tsfm_timestral_attn {
    int32_t is_time;        /* 1: time attention (timeAttention :487-519); 0: variate (:525-544) */
    const float *norm;      /* (d) attn_norms.<i>.scale */
    const float *qkv;       /* (3 d, d) wQKV, rows permuted to (qkv, head, head_dim) (permuteQkv :72-85) */
    const float *out;       /* (d, d) wO */
    const float *gate;      /* (d, d) _gate (sdpa_sigmoid), or NULL */
} tsfm_timestral_attn;

typedef struct tsfm_timestral_layer {
    int32_t n_attn;                 /* 1 or 2, in block_schedule order (config.zig:94-100) */
    tsfm_timestral_attn attn[2];
    const float *mlp_norm;          /* (d) */
    const float *w12;               /* (2 hid, d): gate rows, then up rows (MlpAct :40-46) */
    const float *w3;                /* (d, hid) */
} tsfm_timestral_layer;

typedef struct tsfm_timestral_model {
    int32_t patch, d_model, heads, head_dim, mlp_hidden, n_layers, n_quantiles;
    int32_t block_size, context_length;
    int32_t rope_dim;               /* rotated dims: head_dim * rope_partial_factor (config.zig:34-36) */
    int32_t use_asinh, attend_missing;
    int32_t covariate_enabled;      /* config.covariate_enabled (config.zig:25; true in the reference) */
    float rope_theta, norm_eps, minimum_scale, quantile_width_factor;
    const double *quantile_knots;   /* (n_quantiles) host memory: increasing, containing 0.5 */
    tsfm_resblock patch_proj;       /* 2 patch -> 4 d -> d, act 1 (SiLU), with biases */
    tsfm_resblock head;             /* d -> 4 d -> patch * n_quantiles, act 1, no biases */
    const float *forecast_query;    /* (d) */
    const float *out_norm;          /* (d) */
    const tsfm_timestral_layer *layers;  /* n_layers entries, host memory */
} tsfm_timestral_model;

typedef struct tsfm_timestral_forecast_args {
    tsfm_timestral_model model;
    const float *inputs;            /* (batch, variates, len) */
    const uint8_t *observed;        /* (batch, variates, len): non-zero = observed */
    int32_t batch, variates, len, horizon;   /* variates 1..16 */
    int32_t max_context;            /* Options.max_context; 0 = model.context_length */
    int32_t per_shot_patches;       /* Options.per_shot_horizon_patches; 0 = 32; capped at block_size */
    float quantile_real_cap_k;      /* Options.quantile_real_cap_k (1e4); 0 disables the cap */
    float extreme_value_threshold;  /* Options.extreme_value_threshold (1e30) */
    int32_t symmetric_averaging, clip_nonnegative;  /* Options (both on in the reference) */
    int32_t kv_cache;               /* non-zero: decode over cached K/V (see above) */
    uint32_t flags;                 /* TSFM_ATTN_DEVICE_PTRS, optionally | TSFM_TIMESTRAL_BF16_ATTN
                                       | TSFM_FORECAST_HOST_IO */
    float *out;                     /* (batch, variates, horizon, n_quantiles) */
    void *stream;
    /* Numeric covariates (Covariates.past / .known, src/timestral/forecaster.zig:36-46), NaN =
     * missing; each pointer may be NULL when its count is 0. With known-future covariates every
     * decode block re-encodes the window (context + horizon) as the reference does: kv_cache is
     * ignored (see above); past-only covariates decode over the cache. */
    const float *past;              /* (batch, n_past, len) past-only covariates */
    const float *known;             /* (batch, n_known, len + horizon) known-future covariates */
    int32_t n_past, n_known;        /* variates + n_past + n_known <= TSFM_VARIATE_MAX_ROWS */
} tsfm_timestral_forecast_args;

int tsfm_timestral_forecast(const tsfm_timestral_forecast_args *args);

/* ---------------------------------------------------------------------------------------------
 * Categorical covariates of a Timestral forecast (Covariates.cat_past / .cat_known,
 * src/timestral/forecaster.zig:34-46), encoded into the numeric rows tsfm_timestral_forecast takes,
 * as forecast does before its passes (:86-103): with one target variate each code row is
 * target-encoded against the series' target (encodingTarget :201-217, encodeCategorical
 * :220-238, targetEncode :243-289, slotOf :292-301), otherwise the codes pass through as f32.
 *
 * Encoding target of series s: the forward-filled target from its first observation on, over the
 * last max_context steps of the context (NaN before the first observation and outside the
 * window). Per code row: mean = the mean of the finite target values (0 when none); categories =
 * the distinct finite codes of the context part; a context step whose target is finite adds its
 * target to its category's sum and count (a non-finite code to the missing category's). A context
 * code becomes (mean + sum_c) / (1 + count_c) of its category (non-finite codes: the missing
 * category's), and NaN where both the code and the encoding target are NaN; a future code
 * (steps t .. len-1) becomes its category's value, the missing category's for NaN, and the mean
 * for a code not among the categories. Sums in f64 in step order, the result rounded to f32.
 *
 * The reference appends the encoded rows after the numeric covariate rows of each series
 * (catChannels, :186-195): this call writes code row j of series s to out row s * out_rows + row0
 * + j (len floats each), so a caller builds the combined past / known array in place. Host
 * memory, synchronous, no device needed. Returns TSFM_OK or TSFM_E_INVALID. */
typedef struct tsfm_categorical_args {
    float *out;               /* (batch, out_rows, len) f32 */
    int32_t out_rows, row0;   /* rows per series in out; the first encoded row's index */
    const double *codes;      /* (batch, n_cat, len) category codes, NaN = missing */
    int32_t batch, n_cat;
    int64_t len;              /* t (past codes) or t + horizon (known codes); >= t */
    const float *inputs;      /* (batch, variates, t) targets, zeros where unobserved */
    const uint8_t *observed;  /* (batch, variates, t) */
    int32_t variates;         /* target variates per series (encoding only when 1) */
    int64_t t;                /* context steps */
    int64_t max_context;      /* the forecast's window (its max_context, or the model's
                                 context_length when that is 0); > 0 */
} tsfm_categorical_args;

int tsfm_timestral_encode_categorical(const tsfm_categorical_args *args);

/* ---------------------------------------------------------------------------------------------
 * The reference backend's GEMM seam, with the argument lists and return convention of
 * src/platform/cuda/gemm.c. The reference's binding (src/platform/cuda/gpu.zig:16-44) declares
 * those functions as cuda_*; a HIP binding is the same file with the extern names changed to
 * tsfm_*. nn.linear's weight products
 * (src/core/nn.zig:270-293) and gemmNT (src/core/nn.zig:49-60) then run on the gfx950 matrix cores
 * (the projection kernel, one output, no RoPE).
 *
 * tsfm_weight_register: cuda_weight_register (gemm.c:232-242): a device copy of `len` floats,
 *   NULL on failure. tsfm_weight_release: cuda_weight_release (gemm.c:244-247).
 * tsfm_sgemm_nt: cuda_sgemm_nt (gemm.c:316-322): C[m, n] = alpha * A[m, k] B[n, k]^T, row-major
 *   with leading dimensions; host pointers, synchronous; b_buf = a registered weight (B unused)
 *   or NULL (B uploaded). 0 = done; non-zero = use the CPU. Runs when k % 16 == 0 and n, lda,
 *   ldb, ldc are multiples of 4 (every linear layer of the three families).
 * tsfm_sgemm_nn: cuda_sgemm_nn (gemm.c:324-330): C[m, n] = A[m, k] B[k, n], row-major with leading
 *   dimensions; host pointers, synchronous; b_buf = a registered weight holding B as [k][ldb]
 *   (B unused) or NULL (B uploaded). B is transposed on the device and the product runs on the same
 *   kernel as tsfm_sgemm_nt. Runs when k % 16 == 0 and n, lda, ldc are multiples of 4 (ldb any
 *   >= n). Its caller in the reference is gemmNN (src/core/nn.zig:165-239), the attention's P.V
 *   product, which tsfm_attn_fwd runs inside its kernels; this is the seam for any other. */
void *tsfm_weight_register(const float *data, size_t len);
void tsfm_weight_release(void *handle);
int tsfm_sgemm_nt(int m, int n, int k, float alpha, const float *A, int lda, const float *B, int ldb, float *C,
                  int ldc, void *b_buf);
int tsfm_sgemm_nn(int m, int n, int k, const float *A, int lda, const float *B, int ldb, float *C, int ldc,
                  void *b_buf);

/* ---------------------------------------------------------------------------------------------
 * KV cache for block-autoregressive decode. No counterpart in the reference: Timestral's
 * blockDecode re-encodes the whole grown context every block (src/timestral/forecaster.zig:423-563),
 * recomputing K/V of unchanged prefix tokens. With a causal encoder and a fixed prefix the cached
 * result equals rows [P, P + n) of causal selfAttend over the concatenated sequence.
 * The cache lives in device memory in the layout the decode kernel streams (per (b, h): K rows
 * [pos][D]; V in 32-key chunks transposed for the matrix cores). bf16 and f16 only. */
typedef struct tsfm_kv_cache tsfm_kv_cache;

/* Capacity is rounded up to a multiple of 64 tokens; the cache memory is zero-filled. */
int tsfm_kv_create(tsfm_kv_cache **out, int32_t dtype, int32_t batch, int32_t heads, int32_t head_dim,
                   int32_t capacity);
int tsfm_kv_free(tsfm_kv_cache *cache);
int tsfm_kv_reset(tsfm_kv_cache *cache);
/* Rewind the cache to its first `len` tokens (len <= tsfm_kv_len): a forecast that restarts from
 * the same prefix keeps the prefix's K/V. */
int tsfm_kv_truncate(tsfm_kv_cache *cache, int32_t len);
int32_t tsfm_kv_len(const tsfm_kv_cache *cache);

/* Append n_new tokens to every (b, h): k/v element (b, t, h, c) at b * batch + t * tok + h * D + c.
 * flags/stream as in tsfm_attn_args. */
int tsfm_kv_append(tsfm_kv_cache *cache, const void *k, int64_t k_tok, int64_t k_batch, const void *v,
                   int64_t v_tok, int64_t v_batch, int32_t n_new, uint32_t flags, void *stream);

/* Causal attention of n_q queries over the cached keys [0, tsfm_kv_len): query i sits at key
 * index q_pos0 + i and reads keys 0..=q_pos0+i; requires q_pos0 + n_q <= tsfm_kv_len. */
int tsfm_kv_attend(tsfm_kv_cache *cache, const void *q, int64_t q_tok, int64_t q_batch, void *o,
                   int64_t o_tok, int64_t o_batch, int32_t n_q, int32_t q_pos0, float scale, uint32_t flags,
                   void *stream);

/* One decode block: tsfm_kv_append of the n_new tokens' k/v, then tsfm_kv_attend of their n_new
 * queries at positions len.. (len = tsfm_kv_len before the call), with the same results. With
 * device pointers, n_new == 32 and len a multiple of 32 (Timestral's decode blocks) it is one
 * launch, in which each (series, head) writes its new K/V into the cache and attends; otherwise the
 * two calls run in turn. */
int tsfm_kv_append_attend(tsfm_kv_cache *cache, const void *k, int64_t k_tok, int64_t k_batch, const void *v,
                          int64_t v_tok, int64_t v_batch, const void *q, int64_t q_tok, int64_t q_batch, void *o,
                          int64_t o_tok, int64_t o_batch, int32_t n_new, float scale, uint32_t flags, void *stream);

#ifdef __cplusplus
}
#endif
#endif
