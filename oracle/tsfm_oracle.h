/*
 * tsfm_oracle.h -- CPU oracle for the tsfm-zig attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Results are checked against this library: the parity tests, the
 * smoke check and the CPU-baseline leg of bench.py call it. Product code never
 * links, loads or calls it, and nothing falls back to it.
 *
 * Every function restates one piece of the reference Zig code (path:line under
 * the reference checkout) in C with the same arithmetic: the same operation
 * order, fused multiply-adds exactly where Zig uses @mulAdd, and an ordered
 * lane reduction where Zig uses @reduce(.Add). The SIMD lane count is a
 * compile-time constant (ORC_LANES), as `nn.lanes` is in the reference
 * (src/core/nn.zig:296, std.simd.suggestVectorLength(f32)).
 *
 * How each function is pinned (golden vectors, known-answer tests, closed
 * forms) is listed in tests/test_oracle.py; a function that none of those
 * pins is marked "parity unpinned" below. Currently every exported function
 * has at least one pin.
 */
#ifndef TSFM_ORACLE_H
#define TSFM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* attn.Mask declaration order (src/core/attn.zig:10-21). */
enum { ORC_FULL = 0, ORC_KEYS_ADDITIVE = 1, ORC_CAUSAL = 2, ORC_CAUSAL_KEYS = 3, ORC_FULL_KEYS = 4 };

int orc_lanes(void);

/* nn.expVec, one lane (src/core/nn.zig:344-359). */
float orc_exp_vec(float x);
/* nn.gemmNT builtin path (src/core/nn.zig:49-60, 68-162). */
void orc_gemm_nt(float *cc, size_t ldc, const float *a, size_t lda, const float *b, size_t ldb,
                 size_t m, size_t n, size_t k, float alpha);
/* nn.linear builtin path (src/core/nn.zig:262-293): y = x w^T (+ bias), w (out, in) row-major,
 * output column blocks of 16 over `threads` (par.forRange). */
void orc_linear(size_t threads, float *y, const float *x, size_t rows, const float *w, size_t out, size_t in,
                const float *bias);
/* nn.gemmNN builtin path (src/core/nn.zig:165-239). */
void orc_gemm_nn(float *cc, size_t ldc, const float *a, size_t lda, const float *b, size_t ldb,
                 size_t m, size_t n, size_t k);
/* nn.softmax (src/core/nn.zig:470-505). */
void orc_softmax(float *row, size_t n);
/* nn.dot (src/core/nn.zig:328-340). */
float orc_dot(const float *a, const float *b, size_t n);
/* nn.addInPlace / nn.mulAddInPlace (src/core/nn.zig:302-324). */
void orc_add_in_place(float *dst, const float *src, size_t n);
void orc_mul_add_in_place(float *dst, const float *src, size_t n, float scalar);
/* nn.ropeHalf (src/core/nn.zig:448-467). */
void orc_rope_half(float *x, const float *cos_t, const float *sin_t, size_t half);

/* attn.Mask.pick (src/core/attn.zig:24-28). */
int orc_mask_pick(int causal, int all_keys_valid, int additive);
/* attn.maskedSoftmax (src/core/attn.zig:35-67). key_valid: n bytes (Zig bool). */
void orc_masked_softmax(int mask, float *scores, size_t n, const uint8_t *key_valid);
/* attn.selfAttend (src/core/attn.zig:72-96). st = {q, k, v, o} token strides in floats. */
void orc_self_attend(int mask, float *scores, const float *q, const float *k, const float *v, float *o,
                     const size_t st[4], size_t n, size_t hd, float scale, const uint8_t *key_valid,
                     const float *bias);
/* attn.zig's float64 naive reference (src/core/attn.zig:121-154); o is n x hd, dense. */
void orc_reference_attend_f64(int mask, double *o, const float *q, const float *k, const float *v,
                              const size_t st[4], size_t n, size_t hd, double scale,
                              const uint8_t *key_valid, const float *bias);

/* T5 relative-position bucket (src/chronos_bolt/model.zig:74-85). */
uint32_t orc_relative_bucket(int64_t rel, uint32_t num_buckets, uint32_t max_distance);
/* Model.positionBias (src/chronos_bolt/model.zig:195-205): out (nh, seq, seq) from table (buckets, nh). */
void orc_position_bias(float *out, const float *table, size_t seq, size_t nh, uint32_t num_buckets,
                       uint32_t max_distance);

/* par.forRangeMin over pthreads (src/core/par.zig:18-28). */
typedef void (*orc_range_fn)(const void *ctx, size_t first, size_t last);
void orc_for_range_min(size_t threads, size_t n, size_t min_chunk, const void *ctx, orc_range_fn f);

/* Chronos-Bolt encoder self-attention: forRange(nb*nh, SelfJob.attend)
 * (src/chronos_bolt/model.zig:242-243, 317-346). q/k/v/o are (nb, seq, inner). */
void orc_bolt_self_attention(size_t threads, const float *q, const float *k, const float *v, float *o,
                             const float *bias, const uint8_t *key_valid, int keys_all_valid,
                             size_t nb, size_t seq, size_t inner, size_t nh, size_t hd);
/* Chronos-Bolt decoder cross-attention: forRange(nb*nh, CrossJob.attend)
 * (src/chronos_bolt/model.zig:296-297, 349-381). q/o (nb, inner); k/v (nb, seq, inner). */
void orc_bolt_cross_attention(size_t threads, const float *q, const float *k, const float *v, float *o,
                              const uint8_t *key_valid, size_t nb, size_t seq, size_t inner, size_t nh,
                              size_t hd);

/* Chronos-2 RoPE tables (src/chronos2/model.zig:107-113, 178-187): (seq, hd/2) each. */
void orc_chronos2_rope_tables(float *cos_t, float *sin_t, size_t seq, size_t hd, float theta);
/* Chronos-2 serial RoPE loop over q and k (src/chronos2/model.zig:236-245), in place. */
void orc_chronos2_rope(float *q, float *k, const float *cos_t, const float *sin_t, size_t rows,
                       size_t seq, size_t d, size_t nh, size_t hd);
/* Chronos-2 time attention: forRange(b*nh, TimeJob.attend) (src/chronos2/model.zig:260, 277-309).
 * The model passes scale 1.0 (:306); `scale` is a parameter so other scales can be checked. */
void orc_chronos2_time_attention(size_t threads, const float *q, const float *k, const float *v, float *o,
                                 const uint8_t *key_valid, int keys_all_valid, size_t b, size_t seq,
                                 size_t d, size_t nh, size_t hd, float scale);

/* nn.rmsNorm (src/core/nn.zig:361-396) and nn.relu (:436-444). out may equal x. */
void orc_rms_norm(size_t threads, float *out, const float *x, size_t rows, size_t dim, const float *scale,
                  float eps);
void orc_relu(float *x, size_t n);
/* One Chronos-2 encoder layer's weights (src/chronos2/model.zig Layer), nn.Weight (out, in) layout. */
typedef struct orc_chronos2_layer {
    const float *time_norm, *time_q, *time_k, *time_v, *time_o;
    const float *group_norm, *group_v, *group_o;
    const float *mlp_norm, *mlp_wi, *mlp_wo;
} orc_chronos2_layer;
/* Model.encode (src/chronos2/model.zig:144-206): x (b*seq, d) embedded tokens in, final-normed
 * hidden states out. */
void orc_chronos2_encode(size_t threads, float *x, const uint8_t *key_valid, size_t b, size_t seq, size_t d,
                         size_t nh, size_t hd, size_t d_ff, size_t n_layers, const orc_chronos2_layer *layers,
                         const float *final_norm, float eps, const float *cos_t, const float *sin_t, float scale);
/* ResBlock weights with biases (src/core/resblock.zig:36-61). */
typedef struct orc_resblock {
    const float *hidden_w, *hidden_b, *output_w, *output_b, *residual_w, *residual_b;
    size_t in, hid, out;
} orc_resblock;
/* ResBlock(.relu).forward (src/core/resblock.zig:63-79). */
void orc_resblock_relu(size_t threads, float *y, const float *x, size_t rows, const orc_resblock *rb);
/* The model part of the Chronos-2 forecaster's runChunk (src/chronos2/forecaster.zig:155-183). */
void orc_chronos2_model_forward(size_t threads, float *raw, const float *feats, const float *fut_feats,
                                const uint8_t *ctx_valid, const float *reg, size_t b, size_t n_ctx, size_t n_out,
                                size_t d, size_t nh, size_t hd, size_t d_ff, size_t n_layers,
                                const orc_chronos2_layer *layers, const float *final_norm, float eps,
                                const float *cos_t, const float *sin_t, float scale, const orc_resblock *input_embed,
                                const orc_resblock *output_embed);
/* The Chronos-2 forecaster's runChunk (src/chronos2/forecaster.zig:59-204) around
 * orc_chronos2_model_forward: instance norm, [time_enc, values, mask] patch features, the model,
 * inverse scaling into out (n, horizon, q). Row s is inputs[s * stride + start ..][0..len]. */
void orc_chronos2_forecast(size_t threads, float *out, const float *inputs, size_t stride, size_t start, size_t len,
                           size_t n, size_t ps, size_t horizon, float time_scale, int arcsinh, const float *reg,
                           size_t d, size_t nh, size_t hd, size_t d_ff, size_t n_layers,
                           const orc_chronos2_layer *layers, const float *final_norm, float eps, const float *cos_t,
                           const float *sin_t, float scale, const orc_resblock *input_embed,
                           const orc_resblock *output_embed);
/* Chronos-Bolt layer weights (src/chronos_bolt/model.zig:12-55), nn.Weight (out, in) layout. */
typedef struct orc_bolt_enc_layer {
    const float *attn_norm, *q, *k, *v, *o, *ffn_norm, *wi, *wo;
} orc_bolt_enc_layer;
typedef struct orc_bolt_dec_layer {
    const float *self_norm, *self_v, *self_o, *cross_norm, *cross_q, *cross_k, *cross_v, *cross_o;
    const float *ffn_norm, *wi, *wo;
} orc_bolt_dec_layer;
/* The model part of the Chronos-Bolt forecaster's chunk (src/chronos_bolt/forecaster.zig:199-213). */
void orc_bolt_model_forward(size_t threads, float *raw, const float *feats, const uint8_t *patch_valid,
                            const float *reg, const float *dec_start, const float *rel_table, uint32_t num_buckets,
                            uint32_t max_distance, size_t b, size_t n_patch, size_t d, size_t nh, size_t hd,
                            size_t d_ff, const orc_bolt_enc_layer *enc, size_t n_enc, const float *enc_final_norm,
                            const orc_bolt_dec_layer *dec, size_t n_dec, const float *dec_final_norm, float eps,
                            const orc_resblock *input_embed, const orc_resblock *output_embed);
/* The Chronos-Bolt forecaster's runChunk (src/chronos_bolt/forecaster.zig:130-220). */
void orc_bolt_forecast(size_t threads, float *out, const float *ctx, size_t stride, size_t offset, size_t len,
                       size_t n, size_t ps, float norm_eps, const float *reg, const float *dec_start,
                       const float *rel_table, uint32_t num_buckets, uint32_t max_distance, size_t d, size_t nh,
                       size_t hd, size_t d_ff, const orc_bolt_enc_layer *enc, size_t n_enc,
                       const float *enc_final_norm, const orc_bolt_dec_layer *dec, size_t n_dec,
                       const float *dec_final_norm, float eps, const orc_resblock *input_embed,
                       const orc_resblock *output_embed);
/* The Chronos-Bolt weights and dims, bundled for the forecaster loop. */
typedef struct orc_bolt_model {
    const float *reg, *dec_start, *rel_table;
    uint32_t num_buckets, max_distance;
    size_t d, nh, hd, d_ff;
    const orc_bolt_enc_layer *enc;
    size_t n_enc;
    const float *enc_final_norm;
    const orc_bolt_dec_layer *dec;
    size_t n_dec;
    const float *dec_final_norm;
    float eps;
    const orc_resblock *input_embed, *output_embed;
} orc_bolt_model;
/* quantileLinear (src/chronos_bolt/forecaster.zig:81-92): torch.quantile's linear interpolation
 * of an ascending slice at `level`, ATen's two-sided lerp. */
float orc_quantile_linear(const float *sorted, size_t n, float level);
/* Chronos-Bolt forecaster.forecast (src/chronos_bolt/forecaster.zig:22-78): out (b, horizon, q);
 * inputs (b, t_in), NaN = missing; levels (q) the config's quantiles as f32; P the model's
 * prediction_length (output_embed->out = q * P), max_ctx its context_length. */
void orc_bolt_forecast_horizon(size_t threads, float *out, const float *inputs, size_t b, size_t t_in, size_t horizon,
                               size_t ps, size_t P, size_t max_ctx, const float *levels, size_t q, float norm_eps,
                               const orc_bolt_model *m);
/* Timestral key validity and first observed patch (src/timestral/model.zig:343-362). obs: (rows, w)
 * observation bytes, w = ne * ps; key_valid: (rows, ne) out; first_obs: (rows / vall) out, the first
 * patch with an observation in any row of the group, 0 when the group has none. With
 * attend_missing a patch is valid once any earlier patch of its row was observed. Returns
 * keys_all_valid. */
int orc_timestral_key_valid(uint8_t *key_valid, size_t *first_obs, const uint8_t *obs, size_t rows, size_t vall,
                            size_t ne, size_t ps, int attend_missing);
/* Timestral RoPE tables (src/timestral/model.zig:180-188, 447-463): (groups, sl, hd/2) with
 * sl = ne + h. Encoder token p sits at time p, decoder token j at time l + j, both relative to
 * first_obs[g]; inv_freq is zero past rope_dim / 2 (partial RoPE). */
void orc_timestral_rope_tables(float *cos_t, float *sin_t, size_t groups, size_t ne, size_t l, size_t h,
                               size_t hd, size_t rope_dim, float theta, const size_t *first_obs);
/* Timestral TimeJob.rope (src/timestral/model.zig:558-577), in place on the fused qkv buffer. */
void orc_timestral_rope(size_t threads, float *qkv, const float *cos_t, const float *sin_t, size_t rows,
                        size_t sl, size_t vall, size_t d, size_t nh, size_t hd);
/* Timestral TimeJob.attend (src/timestral/model.zig:580-635). qkv (rows, sl, 3d) in the
 * permuted (token, qkv, head, hd) layout, o (rows, sl, d). bidir: per-row flag (known-future
 * covariate rows), may be NULL. */
void orc_timestral_time_attention(size_t threads, const float *qkv, float *o, const uint8_t *key_valid,
                                  int keys_all_valid, const uint8_t *bidir, size_t rows, size_t ne,
                                  size_t l, size_t h, size_t d, size_t nh, size_t hd);

/* Timestral variate attention (VariateJob.run, src/timestral/model.zig:648-709). qkv (rows*sl, 3d)
 * with rows = groups * vall, o (rows*sl, d), key_valid (rows, ne), roles (vall) in
 * model.Role order (target, past, known); sl = ne + h. */
void orc_timestral_variate_attention(size_t threads, const float *qkv, float *o, const uint8_t *key_valid,
                                     const uint8_t *roles, int cov, size_t groups, size_t vall, size_t ne,
                                     size_t h, size_t d, size_t nh, size_t hd);

/* nn.mulSigmoid (src/core/nn.zig:423-433). */
void orc_mul_sigmoid(float *dst, const float *x, const float *g, size_t n);

/* ---- Timestral model and forecaster (tsfm_oracle_timestral.c), rows that are all targets ---- */
/* nn.siluInPlace, nn.mulSilu, nn.softplus, nn.clampNonfinite (src/core/nn.zig:399-420, 516-563). */
void orc_silu_in_place(float *x, size_t n);
void orc_mul_silu(float *dst, const float *gate, const float *up, size_t n);
float orc_softplus(float x);
void orc_clamp_nonfinite(float *v, size_t n);
/* ResBlock(.silu).forward (src/core/resblock.zig:63-79); bias pointers may be NULL. */
void orc_resblock_silu(size_t threads, float *y, const float *x, size_t rows, const orc_resblock *rb);
/* Model.patchStats / StatsJob (src/timestral/model.zig:210-216, 712-750): per-patch causal float64
 * Welford (loc, scale) of (rows, t) rows, each (rows, t / ps). */
void orc_timestral_patch_stats(size_t threads, float *loc, float *scale, const float *data, const uint8_t *obs,
                               size_t rows, size_t t, size_t ps, double min_scale);
/* One attention of a layer (src/timestral/model.zig:19-33): qkv rows permuted to (qkv, head,
 * head_dim) (permuteQkv, :72-85); gate NULL = no sdpa_sigmoid gate. */
typedef struct orc_timestral_attn {
    int is_time;
    const float *norm, *qkv, *out, *gate;
} orc_timestral_attn;
typedef struct orc_timestral_layer {
    int n_attn;
    orc_timestral_attn attn[2];
    const float *mlp_norm, *w12, *w3; /* w12 (2 hid, d) = [gate; up], w3 (d, hid) */
} orc_timestral_layer;
/* Model (src/timestral/model.zig:126-200) with its config (src/timestral/config.zig:6-45). */
typedef struct orc_timestral_model {
    size_t ps, d, nh, hd, hid, n_layers, q, median, block_size, context_length, rope_dim;
    float rope_theta, norm_eps, quantile_width_factor;
    double minimum_scale;
    int use_asinh, attend_missing;
    const double *knots;                 /* quantile_knots (q) */
    orc_resblock patch_proj, head;       /* ResBlock(.silu): (2 ps -> 4d -> d, biases), (d -> 4d -> ps q) */
    const float *forecast_query, *out_norm;
    const orc_timestral_layer *layers;
} orc_timestral_model;
/* Model.predictBlock (src/timestral/model.zig:220-432) without covariates: ctx/obs (rows, t),
 * rows = groups * vall; out (rows, h * ps, q) quantiles in data units. */
void orc_timestral_predict_block(size_t threads, float *out, const orc_timestral_model *m, const float *ctx,
                                 const uint8_t *obs, size_t t, size_t groups, size_t vall, size_t h);
/* Model.predictBlock with covariates: roles (vall) in model.Role order (0 target, 1 past, 2 known;
 * NULL = all targets), kf/kfm (rows, h * ps) known futures (NULL = blanks); out (groups * targets,
 * h * ps, q). */
void orc_timestral_predict_block_cov(size_t threads, float *out, const orc_timestral_model *m, const float *ctx,
                                     const uint8_t *obs, size_t t, size_t groups, size_t vall, size_t h,
                                     const uint8_t *roles, const float *kf, const uint8_t *kfm);
/* refineBlock (src/timestral/forecaster.zig:582-662) with every row a target: qs (rows, h ps, q) in place. */
void orc_timestral_refine_block(float *qs, const orc_timestral_model *m, const float *ctx, const uint8_t *obs,
                                size_t rows, size_t t, size_t h);
/* forecaster.forecast (src/timestral/forecaster.zig:57-180, forecastRaw :303-421, blockDecode :423-563)
 * without covariates: inputs/observed (b, v, t), out (b, v, horizon, q). max_context 0 = the model's
 * context_length. Returns 0, 1 (a NaN forecast: error.DegenerateInput) or 2 (asymmetric levels). */
/* forecaster.forecast with numeric covariates: past (b, n_past, t), known (b, n_known, t + horizon),
 * NaN = missing; the mirrored pass negates every covariate row. */
int orc_timestral_forecast_cov(size_t threads, float *out, const orc_timestral_model *m, const float *inputs,
                               const uint8_t *observed, size_t b, size_t v, size_t t, size_t horizon,
                               const float *past, size_t n_past, const float *known, size_t n_known,
                               size_t max_context, size_t per_shot, float cap_k, float extreme, int symmetric,
                               int clip_nonnegative);
/* Categorical covariates (src/timestral/forecaster.zig:201-301): codes (b, c, len) f64 -> out (b, c, len) f32. */
void orc_timestral_encode_categorical(float *out, const double *codes, size_t b, size_t c, size_t len,
                                      const float *inputs, const uint8_t *observed, size_t v, size_t t,
                                      size_t max_context);
int orc_timestral_forecast(size_t threads, float *out, const orc_timestral_model *m, const float *inputs,
                           const uint8_t *observed, size_t b, size_t v, size_t t, size_t horizon, size_t max_context,
                           size_t per_shot, float cap_k, float extreme, int symmetric, int clip_nonnegative);

/* Batched selfAttend over (b, h) items with (token, head, dim) layouts: the generic form of
 * the three family jobs above, used by the tests for shapes the families do not fix.
 * q/k/v/o strides: token stride and batch stride in floats; head h at +h*hd. */
void orc_batched_self_attend(size_t threads, int mask, const float *q, size_t q_tok, size_t q_batch,
                             const float *k, size_t k_tok, size_t k_batch, const float *v, size_t v_tok,
                             size_t v_batch, float *o, size_t o_tok, size_t o_batch,
                             const uint8_t *key_valid, size_t kv_batch, const float *bias,
                             size_t nb, size_t nh, size_t n, size_t hd, float scale);

#ifdef __cplusplus
}
#endif
#endif
