// Host-side launchers of the device kernels. Each returns the launch's hipError_t.
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace tsfm {

// f32 q/k/v/o; mask = TSFM_MASK_*, bias = BiasKind.
hipError_t launch_attn_f32(const Params& p, int mask, int bias, bool rope, hipStream_t stream);
hipError_t launch_attn_x3(const Params& p, int mask, int bias, bool rope, hipStream_t stream);

// bf16 (is_bf16) or f16 q/k/v/o, f32 accumulation.
hipError_t launch_attn_half(const Params& p, bool is_bf16, int mask, int bias, bool rope, hipStream_t stream);
// The pipelined half-precision kernel (attn_prefill.hip): masks FULL, CAUSAL, CAUSAL_KEYS and
// FULL_KEYS without bias or RoPE, positive scale. launch_attn_half uses it for those calls.
bool attn_half_pipe_supports(const Params& p, int mask, int bias, bool rope);
hipError_t launch_attn_half_pipe(const Params& p, bool is_bf16, int mask, hipStream_t stream);

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
// The K/V of n_new new tokens, (B, n_new, H*64) with token and batch strides in elements.
struct KvNew {
    const void* k; int64_t k_tok, k_batch;
    const void* v; int64_t v_tok, v_batch;
};
// Block decode in one launch: the n_new tokens' K/V are written at positions pos0.. of the cache,
// and their n_new queries (at the same positions) attend causally over keys [0, pos0 + n_new).
// n_new == kKvFusedBlock and pos0 a multiple of 32 (one workgroup per (series, head), the new
// tokens one 32-key chunk of the cache).
constexpr int kKvFusedBlock = 32;
hipError_t launch_kv_append_attend(const KvLayout& c, bool is_bf16, const KvNew& nw, const void* q, int64_t q_tok,
                                   int64_t q_batch, void* o, int64_t o_tok, int64_t o_batch, int32_t n_new,
                                   int32_t pos0, float scale, hipStream_t stream);

// Timestral variate attention (variate.hip). f32; vall <= 16.
constexpr int kRoleTarget = 0, kRoleKnown = 2;  // model.Role (src/timestral/model.zig:89)
constexpr int kVariateMaxRows = 256;  // rows per series the variate kernels take (kernel-argument roles)
struct VariateParams {
    const float* qkv; int64_t qkv_row, qkv_tok;
    float* o; int64_t o_row, o_tok;
    const float* gate; int64_t gate_row, gate_tok;
    const uint8_t* key_valid; int64_t kv_row;
    uint32_t roles[kVariateMaxRows / 4];  // role of row i in byte i % 4 of word i / 4
    int32_t groups, vall, n_tok, n_enc, heads, cov;
    float scale;
    int32_t heads_per_block, nblk;  // set by launch_variate
    uint32_t qkv_span_bytes;         // set by launch_variate
};
hipError_t launch_variate(const VariateParams& p, hipStream_t stream);

// Fused projection (proj.hip): output sel (0..n_out-1) is y_sel[token, :] = x[token, :] w_sel^T,
// epilogues: kEpiRelu max(y, 0), kEpiSilu y / (1 + exp(-y)), kEpiResidual resid + y (after the bias),
// width columns each (a multiple of 64, or of 4 with a single output); outputs 0 and 1 (q, k)
// get RoPE when rope_cos is set. f32 in (out_dtype:
// 0 f32, 1 bf16, 2 f16 out); d_in a multiple
// of 16, width a multiple of 64, x_tok, y*_tok multiples of 4 and 16-byte aligned pointers.
constexpr int kEpiNone = 0, kEpiRelu = 1, kEpiResidual = 2, kEpiSilu = 3;
struct ProjParams {
    const float* x; int64_t x_tok;
    const float *w0, *w1, *w2, *w3;  // (width, d_in) row-major each, rows w_ld apart
    int64_t w_ld;
    float alpha;                     // result scale (1: none)
    int32_t epi;                     // kEpi*: f32 outputs only
    const float* resid; int64_t resid_tok;  // kEpiResidual: y = resid + x w^T (resid may be y)
    const float* bias;               // per output column, added before the epilogue (one output only)
    void *y0, *y1, *y2, *y3;             // f32, bf16 or f16 elements (out_dtype)
    int64_t y0_tok, y1_tok, y2_tok, y3_tok;
    // Batch strides of the outputs: token t of series row b goes to b * y_batch + t * y_tok
    // (0 = rows packed, b * seq * y_tok). Lets a projection write into a longer per-row buffer.
    int64_t y0_batch, y1_batch, y2_batch, y3_batch;
    const float* rope_cos; const float* rope_sin;
    int64_t rope_table_stride;
    int32_t rope_rows_per_table, rope_row0;
    int32_t tokens, seq, d_in, width, n_out, out_dtype;
    int32_t m_tiles, n_tiles;  // set by launch_proj
    int32_t m_base;            // set by launch_proj: first token of the launch's token tiles
    int32_t chunk;             // set by launch_proj: 16-wide reduction units per accumulation chunk
    int32_t splits, split_steps;  // set by launch_proj: reduction split over workgroups (small products)
    float* partial;               // set by launch_proj: [splits][tokens][width] partial sums
    const void* xp;               // set by launch_proj: x and the weights pre-split into bf16 parts
    const void* wp;               // (PlaneWorkspace), or null: the product splits its own tiles
    // Optional, for products that pass proj_planes_ready: x already split by its producer
    // (launch_rms_norm_planes or another product's y_planes; x is then not read), and / or the
    // result written split (one f32 output, width a multiple of 32, no RoPE) instead of into y0.
    const void* x_pre;
    void* y_planes;
    // Optional row norm of the finished product (one f32 output): norm_out = rmsNorm(y0, norm_scale,
    // norm_eps), the same arithmetic as launch_rms_norm; may be y0 itself.
    const float* norm_scale;
    float* norm_out;
    int64_t norm_out_tok;
    float norm_eps;
    // Optional row norm of the input, for products of at most 16 tokens (the 16-token kernel): x is
    // read as rmsNorm(x, in_norm_scale, in_norm_eps), the same arithmetic as launch_rms_norm.
    const float* in_norm_scale;
    float in_norm_eps;
};
hipError_t launch_proj(const ProjParams& p, hipStream_t stream);
// Whether a product of `tokens` rows (f32 output, no RoPE, no pre-split operands) takes in_norm_scale.
bool proj_fuses_input_norm(int64_t tokens, int64_t d_in);
// Compute units of the current device (looked up once per device; 0 if the query fails).
int device_cus();
// dst[c][r] = src[r][c] for a rows x cols f32 matrix (row strides in elements).
hipError_t launch_transpose_f32(const float* src, int64_t ld_src, float* dst, int64_t ld_dst, int rows, int cols,
                                hipStream_t stream);
// Bytes of split partials launch_proj will need for this product (0: it runs unsplit); sets the
// tiling fields of p as launch_proj does.
size_t proj_split_bytes(ProjParams& p);

// Small products split their reduction over workgroups and sum the partial tiles in a fixed order
// (proj_reduce). The partials go to a device buffer of kSplitWorkspaceBytes that the entry point
// queuing the products provides, for the duration of its call on the calling thread: a
// SplitWorkspace on the stack. The buffer must not be in use by work queued on another stream or
// by another host thread; stream order makes its reuse by consecutive products of one call safe.
// A split product queued with no workspace set fails with hipErrorInvalidValue.
constexpr size_t kSplitWorkspaceBytes = (size_t)1536 * 64 * 64 * sizeof(float);
class SplitWorkspace {
public:
    explicit SplitWorkspace(float* buf);
    ~SplitWorkspace();
    SplitWorkspace(const SplitWorkspace&) = delete;
    SplitWorkspace& operator=(const SplitWorkspace&) = delete;

private:
    float* prev_;
};

// f32 products with d_in a multiple of 32 run on the bf16 matrix cores as three bf16 parts per
// operand. With a PlaneWorkspace set, launch_proj splits x and the weights once per product into
// that buffer (proj_plane_bytes of it) and the product reads the parts from there; without one (or
// with one too small) the product splits its own tiles as it loads them. Both give the same bits.
// Same rules of ownership and lifetime as SplitWorkspace.
size_t proj_plane_bytes(int64_t tokens, int64_t d_in, int64_t n_cols);
// Bytes of one pre-split (rows x cols) operand (cols a multiple of 32), as launch_rms_norm_planes
// and a product's y_planes write it.
size_t plane_operand_bytes(int64_t rows, int64_t cols);
// A product of this shape may take x_pre / y_planes: a PlaneWorkspace holds its weights' parts,
// d_in is a multiple of 32 and the product is large enough to run on pre-split operands.
bool proj_planes_ready(int64_t tokens, int64_t d_in, int64_t n_cols);
// rmsNorm of rows (as launch_rms_norm, the same bits), written split into bf16 parts for a product
// (dim a multiple of 32).
hipError_t launch_rms_norm_planes(const float* x, int64_t x_tok, void* planes, const float* scale, int rows, int dim,
                                  float eps, hipStream_t stream);
class PlaneWorkspace {
public:
    PlaneWorkspace(void* buf, size_t bytes);
    ~PlaneWorkspace();
    PlaneWorkspace(const PlaneWorkspace&) = delete;
    PlaneWorkspace& operator=(const PlaneWorkspace&) = delete;

private:
    void* prev_;
    size_t prev_bytes_;
};

// nn.rmsNorm over rows of dim floats (encoder.hip): dim a multiple of 4, rows 16-byte aligned.
hipError_t launch_rms_norm(const float* x, int64_t x_tok, float* out, int64_t out_tok, const float* scale, int rows,
                           int dim, float eps, hipStream_t stream);
// Chronos-2 sequence [context; REG; future] and its key_valid from the two embeddings, and the
// future tokens' rows back out of it (encoder.hip).
hipError_t launch_assemble_sequence(const float* ctx_emb, const float* fut_emb, const float* reg,
                                    const uint8_t* ctx_valid, float* x, uint8_t* key_valid, int nb, int n_ctx,
                                    int n_out, int d, hipStream_t stream);
hipError_t launch_gather_future(const float* x, float* hidden, int nb, int n_ctx, int n_out, int d,
                                hipStream_t stream);
hipError_t launch_broadcast_rows(const float* v, float* y, int rows, int d, hipStream_t stream);
// Chronos-Bolt forecaster's per-series instance norm + patch features, and the inverse norm (encoder.hip).
hipError_t launch_bolt_prepare(const float* ctx, int64_t stride, int64_t offset, int len, int ps, int n_patch, int pad,
                               float norm_eps, float* feats, uint8_t* patch_valid, float* loc, float* scale, int n,
                               hipStream_t stream);
hipError_t launch_chronos2_prepare(const float* inputs, int64_t stride, int64_t start, int len, int ps, int n_ctx,
                                  int n_out, int pad, float tscale, int arcsinh, float* feats, float* fut_feats,
                                  uint8_t* ctx_valid, float* loc, float* scale, int n, hipStream_t stream);
hipError_t launch_chronos2_finish(const float* raw, const float* loc, const float* scale, float* out, int n, int n_out,
                                  int q, int ps, int horizon, int arcsinh, hipStream_t stream);
hipError_t launch_bolt_finish(const float* raw, const float* loc, const float* scale, float* out, int n, int per,
                              hipStream_t stream);

// ---- Chronos-Bolt long horizons (bolt_horizon.hip) ----
struct BoltLevels {
    float v[16];
};
// pred (b, q, P) -> steps [start, start + P) of out (b, horizon, q).
hipError_t launch_bolt_store_block(const float* pred, int b, int q, int P, int horizon, int start, float* out,
                                   hipStream_t s);
// dst (rows, new_len): row r = the last new_len steps of (src row r / rep ++ pred row r).
hipError_t launch_bolt_window(const float* src, int64_t src_stride, int64_t src_off, int len, int rep,
                              const float* pred, int P, float* dst, int new_len, int rows, hipStream_t s);
// raw (b * q, q, P) -> pred (b, q, P): the q levels of the q * q samples of each (series, step).
hipError_t launch_bolt_sample_quantiles(const float* raw, int b, int q, int P, const BoltLevels& lv, float* pred,
                                        hipStream_t s);

// ---- Timestral forecaster pieces (timestral.hip) ----
struct TsStatsParams {
    const float* ctx;
    const uint8_t* mask;
    int cap_t, cap_p, rows, ps, from, t, attend_missing;
    double min_scale;
    float *loc, *scale;
    uint8_t* key_valid;
    int* row_first;
    double *state, *fold;  // (rows, 4) Welford of StatsJob, (rows, 3) refineBlock's patch fold
};
struct TsRope {
    float inv_freq[32];  // model.zig:180-188: zero past rope_dim / 2
};
struct TsHead {
    int ps, q, median, use_asinh;
    float wf;          // quantile_width_factor
    float widths[32];  // knot widths (model.zig:392-395), q <= 32
};
// forecastRaw's rows: groups of vall rows (V targets, n_past past-only, n_known known-future
// covariates), groups >= batch the mirrored pass.
struct TsContextParams {
    const float* inputs;
    const uint8_t* observed;
    const float* past;   // (batch, n_past, t0), NaN = missing
    const float* known;  // (batch, n_known, t0 + horizon), NaN = missing
    int batch, V, n_past, n_known, vall, rows, t0, keep, t, horizon, hpad, cap_t;
    float* ctx;
    uint8_t* mask;
    float* kf;     // (rows, hpad) known-future values
    uint8_t* kfm;  // (rows, hpad) their observation flags
    uint8_t* nonneg;
};
hipError_t launch_ts_context(const TsContextParams& p, hipStream_t s);
hipError_t launch_ts_window(float* ctx, uint8_t* mask, int cap_t, int t, int blen, const float* kf, const uint8_t* kfm,
                            int hpad, int done, int vall, int known_from, int rows, hipStream_t s);
hipError_t launch_ts_known_stats(const float* ctx, const uint8_t* mask, int cap_t, int w, int ps, int rows, int vall,
                                 int known_from, float min_scale, float* loc, float* scale, int cap_p,
                                 uint8_t* no_asinh, hipStream_t s);
hipError_t launch_ts_stats(const TsStatsParams& p, hipStream_t s);
hipError_t launch_ts_features(const float* ctx, const uint8_t* mask, int cap_t, const float* loc, const float* scale,
                              int cap_p, int rows, int p0, int l, int ps, int use_asinh, const uint8_t* no_asinh,
                              float* feats, hipStream_t s);
hipError_t launch_ts_rope_tables(const int* row_first, int groups, int vall, int n_tok, int ne, int shift,
                                 const TsRope& rp, float* cos_t, float* sin_t, int* first_obs, hipStream_t s);
hipError_t launch_ts_assemble(const float* emb, const float* query, float* x, int rows, int m, int h, int d,
                              hipStream_t s);
hipError_t launch_ts_mul_sigmoid(float* o, const float* g, int64_t n, hipStream_t s);
// o = f32(oh) for n bf16 elements (n % 4 == 0), then o / (1 + exp(-g)) when g is given.
hipError_t launch_ts_from_bf16(const uint16_t* oh, const float* g, float* o, int64_t n, hipStream_t s);
hipError_t launch_ts_mul_silu(const float* hbuf, float* a, int64_t tokens, int hid, hipStream_t s);
hipError_t launch_ts_head_finish(const float* raw, const float* loc, const float* scale, int cap_p, int l, int rows,
                                 int h, const TsHead& hp, float* qs, hipStream_t s);
hipError_t launch_ts_refine(float* qs, const float* loc, const float* scale, int cap_p, int l, const double* fold,
                            int rows, int h, int ps, int q, int median, double min_scale, float* frames,
                            hipStream_t s);
hipError_t launch_ts_store_block(const float* qs, int rows, int batch, int vall, int V, int blen, int done, int horizon,
                                 int q, float* out, float* mir, hipStream_t s);
hipError_t launch_ts_feedback(const float* qs, int rows, int vall, int V, int blen, int q, int median, float extreme,
                              float* ctx, uint8_t* mask, int cap_t, int t, hipStream_t s);
hipError_t launch_ts_slide(const float* src, const uint8_t* src_mask, float* dst, uint8_t* dst_mask, int rows,
                           int cap_t, int start, int keep, hipStream_t s);
hipError_t launch_ts_cap_bounds(const float* ctx, const uint8_t* mask, int cap_t, int t, int ps, const float* scale,
                                int cap_p, int rows, float cap_k, float* bounds, hipStream_t s);
hipError_t launch_ts_final(float* out, const float* mir, const float* bounds, const uint8_t* nonneg, int R, int V,
                           int vall, int horizon, int q, int cap, int symmetric, int clip, hipStream_t s);

}  // namespace tsfm
