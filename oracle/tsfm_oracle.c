/*
 * tsfm_oracle.c -- CPU oracle for the tsfm-zig attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: what the HIP kernels are checked against, and the CPU
 * baseline that bench.py times beside them. Product code never calls it.
 *
 * A C restatement of the reference's builtin CPU path (`-Dblas=builtin`, the
 * Linux default, build.zig:11-12). Arithmetic follows the Zig source:
 *   - Zig does not contract `a * b + c`; this file is compiled with
 *     -ffp-contract=off and uses fmaf() exactly where Zig calls @mulAdd;
 *   - @reduce(.Add, v) on floats keeps associativity (strict float mode), i.e.
 *     an ordered sum over lanes 0..L-1, restated by red_add();
 *   - @round is round-half-away-from-zero (roundf); @exp/@log/@cos/@sin of f32
 *     are libm's expf/logf/cosf/sinf; std.math.pow(f32) is powf.
 * The lane count L = ORC_LANES is fixed at compile time like nn.lanes
 * (src/core/nn.zig:296).
 */
#include "tsfm_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#ifndef ORC_LANES
#define ORC_LANES 8
#endif
#define L ORC_LANES

int orc_lanes(void) { return L; }

/* Ordered lane sum: @reduce(.Add, v) with associativity preserved. */
static inline float red_add(const float *v) {
    float s = v[0];
    for (int e = 1; e < L; e++) s += v[e];
    return s;
}

/* ------------------------------------------------------------------------------------------ */
/* nn.expVec (src/core/nn.zig:344-359): Cephes expf, clamp + range reduction + degree-6 poly. */

float orc_exp_vec(float x_in) {
    float x = x_in;
    if (x < -87.33654f) x = -87.33654f; /* @max(x_in, -87.33654) */
    if (x > 88.72284f) x = 88.72284f;   /* @min(.., 88.72284) */
    const float fx = roundf(x * 1.44269504088896341f);
    float r = x - fx * 0.693359375f;
    r = r - fx * -2.12194440e-4f;
    float y = 1.9875691500e-4f;
    y = y * r + 1.3981999507e-3f;
    y = y * r + 8.3334519073e-3f;
    y = y * r + 4.1665795894e-2f;
    y = y * r + 1.6666665459e-1f;
    y = y * r + 5.0000001201e-1f;
    y = y * r * r + r + 1.0f;
    const int32_t n = (int32_t)fx;
    const uint32_t bits = (uint32_t)(n + 127) << 23;
    float pow2;
    memcpy(&pow2, &bits, sizeof pow2);
    return y * pow2;
}

/* ------------------------------------------------------------------------------------------ */
/* nn.gemmNTFallback builtin path (src/core/nn.zig:68-162). Register tile of row_tile rows of A
 * against 4 rows of B; each output is an @mulAdd chain per lane, an ordered lane sum, then the
 * k % L tail added unfused, then scaled by alpha. */

#define RT ((L > 4) ? 2 : 4)

void orc_gemm_nt(float *cc, size_t ldc, const float *a, size_t lda, const float *b, size_t ldb,
                 size_t m, size_t n, size_t k, float alpha) {
    const size_t kv = k / L * L;
    size_t i = 0;
    for (; i + RT <= m; i += RT) {
        size_t j = 0;
        for (; j + 4 <= n; j += 4) {
            float acc[RT][4][L];
            memset(acc, 0, sizeof acc);
            for (size_t p = 0; p < kv; p += L)
                for (int u = 0; u < RT; u++)
                    for (int w = 0; w < 4; w++)
                        for (int e = 0; e < L; e++)
                            acc[u][w][e] = fmaf(a[(i + u) * lda + p + e], b[(j + w) * ldb + p + e], acc[u][w][e]);
            for (int u = 0; u < RT; u++)
                for (int w = 0; w < 4; w++) {
                    float sum = red_add(acc[u][w]);
                    for (size_t q = kv; q < k; q++) sum += a[(i + u) * lda + q] * b[(j + w) * ldb + q];
                    cc[(i + u) * ldc + j + w] = alpha * sum;
                }
        }
        for (; j < n; j++) { /* column remainder */
            float acc[RT][L];
            memset(acc, 0, sizeof acc);
            for (size_t p = 0; p < kv; p += L)
                for (int u = 0; u < RT; u++)
                    for (int e = 0; e < L; e++)
                        acc[u][e] = fmaf(a[(i + u) * lda + p + e], b[j * ldb + p + e], acc[u][e]);
            for (int u = 0; u < RT; u++) {
                float sum = red_add(acc[u]);
                for (size_t q = kv; q < k; q++) sum += a[(i + u) * lda + q] * b[j * ldb + q];
                cc[(i + u) * ldc + j] = alpha * sum;
            }
        }
    }
    for (; i < m; i++) { /* row remainder */
        const float *ar = a + i * lda;
        size_t j = 0;
        for (; j + 4 <= n; j += 4) {
            float acc[4][L];
            memset(acc, 0, sizeof acc);
            for (size_t p = 0; p < kv; p += L)
                for (int u = 0; u < 4; u++)
                    for (int e = 0; e < L; e++)
                        acc[u][e] = fmaf(ar[p + e], b[(j + u) * ldb + p + e], acc[u][e]);
            for (int u = 0; u < 4; u++) {
                float sum = red_add(acc[u]);
                for (size_t q = kv; q < k; q++) sum += ar[q] * b[(j + u) * ldb + q];
                cc[i * ldc + j + u] = alpha * sum;
            }
        }
        for (; j < n; j++) {
            float acc[L];
            memset(acc, 0, sizeof acc);
            for (size_t p = 0; p < kv; p += L)
                for (int e = 0; e < L; e++) acc[e] = fmaf(ar[p + e], b[j * ldb + p + e], acc[e]);
            float sum = red_add(acc);
            for (size_t q = kv; q < k; q++) sum += ar[q] * b[j * ldb + q];
            cc[i * ldc + j] = alpha * sum;
        }
    }
}

/* nn.gemmNN builtin path (src/core/nn.zig:179-238): four rows of A share each row of B; a k index
 * whose four A values are all exactly zero is skipped (`:196`), a single remainder row skips its
 * zeros (`:227`). Accumulation is `c + a * b`, unfused, in increasing k. */
void orc_gemm_nn(float *cc, size_t ldc, const float *a, size_t lda, const float *b, size_t ldb,
                 size_t m, size_t n, size_t k) {
    size_t i = 0;
    for (; i + 4 <= m; i += 4) {
        float *c0 = cc + (i + 0) * ldc, *c1 = cc + (i + 1) * ldc;
        float *c2 = cc + (i + 2) * ldc, *c3 = cc + (i + 3) * ldc;
        memset(c0, 0, n * sizeof(float));
        memset(c1, 0, n * sizeof(float));
        memset(c2, 0, n * sizeof(float));
        memset(c3, 0, n * sizeof(float));
        for (size_t p = 0; p < k; p++) {
            const float a0 = a[(i + 0) * lda + p], a1 = a[(i + 1) * lda + p];
            const float a2 = a[(i + 2) * lda + p], a3 = a[(i + 3) * lda + p];
            if (a0 == 0 && a1 == 0 && a2 == 0 && a3 == 0) continue;
            const float *brow = b + p * ldb;
            for (size_t j = 0; j < n; j++) {
                const float bv = brow[j];
                c0[j] = c0[j] + a0 * bv;
                c1[j] = c1[j] + a1 * bv;
                c2[j] = c2[j] + a2 * bv;
                c3[j] = c3[j] + a3 * bv;
            }
        }
    }
    for (; i < m; i++) {
        float *crow = cc + i * ldc;
        memset(crow, 0, n * sizeof(float));
        for (size_t p = 0; p < k; p++) {
            const float av = a[i * lda + p];
            if (av == 0) continue;
            const float *brow = b + p * ldb;
            for (size_t j = 0; j < n; j++) crow[j] = crow[j] + av * brow[j];
        }
    }
}

/* ------------------------------------------------------------------------------------------ */
/* nn.softmax (src/core/nn.zig:470-505): lane-wise max, then expVec over whole vectors and @exp
 * over the tail, -inf mapped to exactly 0, a lane-wise partial sum reduced in order, then every
 * entry multiplied by 1/sum. */
void orc_softmax(float *row, size_t n) {
    const float ninf = -INFINITY;
    float mxv[L];
    for (int e = 0; e < L; e++) mxv[e] = ninf;
    size_t i = 0;
    for (; i + L <= n; i += L)
        for (int e = 0; e < L; e++) mxv[e] = fmaxf(mxv[e], row[i + e]);
    float mx = mxv[0];
    for (int e = 1; e < L; e++) mx = fmaxf(mx, mxv[e]);
    for (; i < n; i++) mx = fmaxf(mx, row[i]);

    float sumv[L];
    memset(sumv, 0, sizeof sumv);
    i = 0;
    for (; i + L <= n; i += L)
        for (int e = 0; e < L; e++) {
            const float v = row[i + e];
            const float ev = (v == ninf) ? 0.0f : orc_exp_vec(v - mx);
            row[i + e] = ev;
            sumv[e] += ev;
        }
    float sum = red_add(sumv);
    for (; i < n; i++) {
        row[i] = (row[i] == ninf) ? 0.0f : expf(row[i] - mx);
        sum += row[i];
    }
    const float inv = 1.0f / sum;
    for (i = 0; i < n; i++) row[i] *= inv;
}

/* nn.dot (src/core/nn.zig:328-340): `acc += av * bv` (unfused) per lane, ordered lane sum, tail. */
float orc_dot(const float *a, const float *b, size_t n) {
    float acc[L];
    memset(acc, 0, sizeof acc);
    size_t i = 0;
    for (; i + L <= n; i += L)
        for (int e = 0; e < L; e++) acc[e] += a[i + e] * b[i + e];
    float sum = red_add(acc);
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

void orc_add_in_place(float *dst, const float *src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = dst[i] + src[i];
}

void orc_mul_add_in_place(float *dst, const float *src, size_t n, float scalar) {
    for (size_t i = 0; i < n; i++) dst[i] = dst[i] + scalar * src[i];
}

/* nn.ropeHalf (src/core/nn.zig:448-467): pairs (i, i + half), unfused products. */
void orc_rope_half(float *x, const float *cos_t, const float *sin_t, size_t half) {
    float *lo = x, *hi = x + half;
    for (size_t i = 0; i < half; i++) {
        const float x1 = lo[i], x2 = hi[i];
        lo[i] = x1 * cos_t[i] - x2 * sin_t[i];
        hi[i] = x2 * cos_t[i] + x1 * sin_t[i];
    }
}

/* ------------------------------------------------------------------------------------------ */
/* attn.zig */

int orc_mask_pick(int causal, int all_keys_valid, int additive) {
    if (all_keys_valid) return causal ? ORC_CAUSAL : ORC_FULL;
    if (causal) return ORC_CAUSAL_KEYS;
    return additive ? ORC_KEYS_ADDITIVE : ORC_FULL_KEYS;
}

void orc_masked_softmax(int mask, float *scores, size_t n, const uint8_t *key_valid) {
    switch (mask) {
    case ORC_FULL:
        for (size_t i = 0; i < n; i++) orc_softmax(scores + i * n, n);
        break;
    case ORC_KEYS_ADDITIVE: {
        const float mask_min = -FLT_MAX;
        for (size_t i = 0; i < n; i++) {
            float *row = scores + i * n;
            for (size_t j = 0; j < n; j++)
                if (!key_valid[j]) row[j] += mask_min;
            orc_softmax(row, n);
        }
        break;
    }
    case ORC_CAUSAL:
        for (size_t i = 0; i < n; i++) {
            orc_softmax(scores + i * n, i + 1);
            memset(scores + i * n + i + 1, 0, (n - i - 1) * sizeof(float));
        }
        break;
    case ORC_CAUSAL_KEYS:
    case ORC_FULL_KEYS:
        for (size_t i = 0; i < n; i++) {
            float *row = scores + i * n;
            for (size_t j = 0; j < n; j++) {
                const int allowed = j == i || (key_valid[j] && (mask == ORC_FULL_KEYS || j <= i));
                if (!allowed) row[j] = -INFINITY;
            }
            orc_softmax(row, n);
        }
        break;
    default:
        break;
    }
}

void orc_self_attend(int mask, float *scores, const float *q, const float *k, const float *v, float *o,
                     const size_t st[4], size_t n, size_t hd, float scale, const uint8_t *key_valid,
                     const float *bias) {
    orc_gemm_nt(scores, n, q, st[0], k, st[1], n, n, hd, scale);
    if (bias) orc_add_in_place(scores, bias, n * n);
    orc_masked_softmax(mask, scores, n, key_valid);
    orc_gemm_nn(o, st[3], scores, n, v, st[2], n, hd, n);
}

/* allowedRef (src/core/attn.zig:122-130). */
static int allowed_ref(int mask, const uint8_t *kv, size_t i, size_t j) {
    switch (mask) {
    case ORC_FULL: return 1;
    case ORC_KEYS_ADDITIVE: return kv[j] != 0;
    case ORC_CAUSAL: return j <= i;
    case ORC_CAUSAL_KEYS: return j == i || (kv[j] && j <= i);
    case ORC_FULL_KEYS: return j == i || kv[j];
    default: return 0;
    }
}

void orc_reference_attend_f64(int mask, double *o, const float *q, const float *k, const float *v,
                              const size_t st[4], size_t n, size_t hd, double scale,
                              const uint8_t *key_valid, const float *bias) {
    double *s = (double *)malloc((n ? n : 1) * sizeof(double));
    for (size_t i = 0; i < n; i++) {
        double mx = -INFINITY;
        for (size_t j = 0; j < n; j++) {
            double dot = 0;
            for (size_t c = 0; c < hd; c++) dot += (double)q[i * st[0] + c] * (double)k[j * st[1] + c];
            s[j] = dot * scale + (bias ? (double)bias[i * n + j] : 0.0);
            if (allowed_ref(mask, key_valid, i, j)) mx = fmax(mx, s[j]);
        }
        double z = 0;
        for (size_t j = 0; j < n; j++) {
            s[j] = allowed_ref(mask, key_valid, i, j) ? exp(s[j] - mx) : 0.0;
            z += s[j];
        }
        for (size_t c = 0; c < hd; c++) {
            double acc = 0;
            for (size_t j = 0; j < n; j++) acc += s[j] / z * (double)v[j * st[2] + c];
            o[i * hd + c] = acc;
        }
    }
    free(s);
}

/* ------------------------------------------------------------------------------------------ */
/* Chronos-Bolt (src/chronos_bolt/model.zig) */

uint32_t orc_relative_bucket(int64_t rel, uint32_t num_buckets, uint32_t max_distance) {
    const uint32_t half = num_buckets / 2;
    const uint32_t base = rel > 0 ? half : 0;
    const uint32_t rp = (uint32_t)(rel < 0 ? -rel : rel);
    const uint32_t max_exact = half / 2;
    if (rp < max_exact) return base + rp;
    const float ratio = (float)rp / (float)max_exact;
    const float denom = (float)log((double)max_distance / (double)max_exact);
    const float large_f = logf(ratio) / denom * (float)(half - max_exact);
    const uint32_t large = max_exact + (uint32_t)large_f;
    return base + (large < half - 1 ? large : half - 1);
}

void orc_position_bias(float *out, const float *table, size_t seq, size_t nh, uint32_t num_buckets,
                       uint32_t max_distance) {
    for (size_t i = 0; i < seq; i++)
        for (size_t j = 0; j < seq; j++) {
            const int64_t rel = (int64_t)j - (int64_t)i;
            const uint32_t bucket = orc_relative_bucket(rel, num_buckets, max_distance);
            for (size_t h = 0; h < nh; h++) out[h * seq * seq + i * seq + j] = table[bucket * nh + h];
        }
}

/* ------------------------------------------------------------------------------------------ */
/* par.forRangeMin (src/core/par.zig:18-28) on pthreads: contiguous chunks, the first one on the
 * calling thread. */

typedef struct {
    const void *ctx;
    orc_range_fn f;
    size_t first, last;
} range_task;

static void *range_thread(void *p) {
    range_task *t = (range_task *)p;
    t->f(t->ctx, t->first, t->last);
    return NULL;
}

void orc_for_range_min(size_t threads, size_t n, size_t min_chunk, const void *ctx, orc_range_fn f) {
    if (min_chunk == 0) min_chunk = 1;
    size_t chunks = (n + min_chunk - 1) / min_chunk;
    if (threads < chunks) chunks = threads;
    if (chunks <= 1) {
        f(ctx, 0, n);
        return;
    }
    const size_t size = (n + chunks - 1) / chunks;
    size_t ntasks = 0;
    for (size_t start = size; start < n; start += size) ntasks++;
    pthread_t *tid = (pthread_t *)calloc(ntasks ? ntasks : 1, sizeof(pthread_t));
    range_task *tasks = (range_task *)calloc(ntasks ? ntasks : 1, sizeof(range_task));
    int *started = (int *)calloc(ntasks ? ntasks : 1, sizeof(int));
    size_t t = 0;
    for (size_t start = size; start < n; start += size, t++) {
        tasks[t] = (range_task){ctx, f, start, start + size < n ? start + size : n};
        /* Io.async runs the task inline when no thread is free; do the same if creation fails. */
        if (pthread_create(&tid[t], NULL, range_thread, &tasks[t]) == 0) started[t] = 1;
        else range_thread(&tasks[t]);
    }
    f(ctx, 0, size < n ? size : n);
    for (t = 0; t < ntasks; t++)
        if (started[t]) pthread_join(tid[t], NULL);
    free(started);
    free(tasks);
    free(tid);
}

/* nn.linear on the builtin CPU path (src/core/nn.zig:262-293): y[rows, out] = x[rows, in] w^T
 * (+ bias). Products with rows*out*in >= 2^20 and out >= 2*col_block split their output columns
 * into blocks of col_block = 16 over the pool (linearBlocks, :264-267); each block is linearCols
 * (:250-256): gemmNTWeight = gemmNTFallback over the block's contiguous weight rows, then the bias. */
typedef struct {
    float *y;
    const float *x;
    size_t rows;
    const float *w;
    size_t out, in;
    const float *bias;
} linear_ctx;

static void linear_cols(const linear_ctx *c, size_t j0, size_t j1) {
    orc_gemm_nt(c->y + j0, c->out, c->x, c->in, c->w + j0 * c->in, c->in, c->rows, j1 - j0, c->in, 1.0f);
    if (c->bias)
        for (size_t r = 0; r < c->rows; r++) orc_add_in_place(c->y + r * c->out + j0, c->bias + j0, j1 - j0);
}

static void linear_blocks(const void *ctx, size_t b0, size_t b1) {
    const linear_ctx *c = (const linear_ctx *)ctx;
    const size_t col_block = 16, nblocks = (c->out + col_block - 1) / col_block;
    linear_cols(c, b0 * col_block, b1 == nblocks ? c->out : b1 * col_block);
}

void orc_linear(size_t threads, float *y, const float *x, size_t rows, const float *w, size_t out, size_t in,
                const float *bias) {
    const linear_ctx c = {y, x, rows, w, out, in, bias};
    if (rows * out * in >= ((size_t)1 << 20) && out >= 2 * 16)
        orc_for_range_min(threads, (out + 15) / 16, 1, &c, linear_blocks);
    else
        linear_cols(&c, 0, out);
}

/* SelfJob.attend (src/chronos_bolt/model.zig:331-345). */
typedef struct {
    const float *q, *k, *v;
    float *o;
    const float *bias;
    const uint8_t *key_valid;
    int keys_all_valid;
    size_t seq, inner, nh, hd;
} bolt_self_job;

static void bolt_self_attend(const void *p, size_t first, size_t last) {
    const bolt_self_job *j = (const bolt_self_job *)p;
    const size_t seq = j->seq;
    float *scores = (float *)malloc(seq * seq * sizeof(float));
    const int mask = orc_mask_pick(0, j->keys_all_valid, 1);
    const size_t st[4] = {j->inner, j->inner, j->inner, j->inner};
    for (size_t item = first; item < last; item++) {
        const size_t r = item / j->nh, h = item % j->nh;
        const size_t off = r * seq * j->inner + h * j->hd;
        orc_self_attend(mask, scores, j->q + off, j->k + off, j->v + off, j->o + off, st, seq, j->hd, 1.0f,
                        j->key_valid + r * seq, j->bias + h * seq * seq);
    }
    free(scores);
}

void orc_bolt_self_attention(size_t threads, const float *q, const float *k, const float *v, float *o,
                             const float *bias, const uint8_t *key_valid, int keys_all_valid,
                             size_t nb, size_t seq, size_t inner, size_t nh, size_t hd) {
    const bolt_self_job job = {q, k, v, o, bias, key_valid, keys_all_valid, seq, inner, nh, hd};
    orc_for_range_min(threads, nb * nh, 1, &job, bolt_self_attend);
}

/* CrossJob.attend (src/chronos_bolt/model.zig:360-380). */
typedef struct {
    const float *q, *k, *v;
    float *o;
    const uint8_t *key_valid;
    size_t seq, inner, nh, hd;
} bolt_cross_job;

static void bolt_cross_attend(const void *p, size_t first, size_t last) {
    const bolt_cross_job *j = (const bolt_cross_job *)p;
    const size_t seq = j->seq, hd = j->hd;
    const float mask_min = -FLT_MAX;
    float *scores = (float *)malloc(seq * sizeof(float));
    for (size_t item = first; item < last; item++) {
        const size_t r = item / j->nh, h = item % j->nh;
        const float *qh = j->q + r * j->inner + h * hd;
        for (size_t t = 0; t < seq; t++) {
            const float *kh = j->k + (r * seq + t) * j->inner + h * hd;
            scores[t] = orc_dot(qh, kh, hd);
            if (!j->key_valid[r * seq + t]) scores[t] += mask_min;
        }
        orc_softmax(scores, seq);
        float *oh = j->o + r * j->inner + h * hd;
        memset(oh, 0, hd * sizeof(float));
        for (size_t t = 0; t < seq; t++)
            orc_mul_add_in_place(oh, j->v + (r * seq + t) * j->inner + h * hd, hd, scores[t]);
    }
    free(scores);
}

void orc_bolt_cross_attention(size_t threads, const float *q, const float *k, const float *v, float *o,
                              const uint8_t *key_valid, size_t nb, size_t seq, size_t inner, size_t nh,
                              size_t hd) {
    const bolt_cross_job job = {q, k, v, o, key_valid, seq, inner, nh, hd};
    orc_for_range_min(threads, nb * nh, 1, &job, bolt_cross_attend);
}

/* ------------------------------------------------------------------------------------------ */
/* Chronos-2 (src/chronos2/model.zig) */

void orc_chronos2_rope_tables(float *cos_t, float *sin_t, size_t seq, size_t hd, float theta) {
    const size_t half = hd / 2;
    float *inv_freq = (float *)malloc((half ? half : 1) * sizeof(float));
    for (size_t i = 0; i < half; i++) {
        const float idx = (float)(2 * i);
        inv_freq[i] = 1.0f / powf(theta, idx / (float)hd);
    }
    for (size_t tok = 0; tok < seq; tok++) {
        const float pos = (float)tok;
        for (size_t i = 0; i < half; i++) {
            const float ang = inv_freq[i] * pos;
            cos_t[tok * half + i] = cosf(ang);
            sin_t[tok * half + i] = sinf(ang);
        }
    }
    free(inv_freq);
}

void orc_chronos2_rope(float *q, float *k, const float *cos_t, const float *sin_t, size_t rows,
                       size_t seq, size_t d, size_t nh, size_t hd) {
    const size_t half = hd / 2;
    for (size_t r = 0; r < rows; r++) {
        const size_t tok = r % seq;
        const float *cs = cos_t + tok * half, *sn = sin_t + tok * half;
        for (size_t hh = 0; hh < nh; hh++) {
            const size_t off = r * d + hh * hd;
            orc_rope_half(q + off, cs, sn, half);
            orc_rope_half(k + off, cs, sn, half);
        }
    }
}

typedef struct {
    const float *q, *k, *v;
    float *o;
    const uint8_t *key_valid;
    int keys_all_valid;
    size_t seq, d, nh, hd;
    float scale;
} c2_time_job;

static void c2_time_attend(const void *p, size_t first, size_t last) {
    const c2_time_job *j = (const c2_time_job *)p;
    const size_t seq = j->seq, d = j->d, hd = j->hd;
    float *scores = (float *)malloc(seq * seq * sizeof(float));
    const size_t st[4] = {d, d, d, d};
    for (size_t item = first; item < last; item++) {
        const size_t r = item / j->nh, hh = item % j->nh;
        const size_t off = hh * hd, base = r * seq * d;
        const int mask = orc_mask_pick(0, j->keys_all_valid, 1);
        orc_self_attend(mask, scores, j->q + base + off, j->k + base + off, j->v + base + off,
                        j->o + base + off, st, seq, hd, j->scale, j->key_valid + r * seq, NULL);
    }
    free(scores);
}

void orc_chronos2_time_attention(size_t threads, const float *q, const float *k, const float *v, float *o,
                                 const uint8_t *key_valid, int keys_all_valid, size_t b, size_t seq,
                                 size_t d, size_t nh, size_t hd, float scale) {
    const c2_time_job job = {q, k, v, o, key_valid, keys_all_valid, seq, d, nh, hd, scale};
    orc_for_range_min(threads, b * nh, 1, &job, c2_time_attend);
}

/* nn.rmsNorm (src/core/nn.zig:361-396): per row, a lane-parallel sum of squares (multiply, then
 * add: no fused multiply-add in the Zig), an ordered lane reduce, the scalar tail, then
 * inv = 1 / sqrt(ss / dim + eps) and out = x * inv * scale, left to right. Rows split over the pool
 * in chunks of at least 64 (par.forRangeMin), which does not change the result. */
typedef struct {
    float *out;
    const float *x;
    size_t dim;
    const float *scale;
    float eps;
} norm_ctx;

static void rms_norm_rows(const void *p, size_t r0, size_t r1) {
    const norm_ctx *c = (const norm_ctx *)p;
    const size_t dim = c->dim;
    for (size_t r = r0; r < r1; r++) {
        const float *xr = c->x + r * dim;
        float acc[L];
        for (int e = 0; e < L; e++) acc[e] = 0.f;
        size_t i = 0;
        for (; i + L <= dim; i += L)
            for (int e = 0; e < L; e++) {
                const float sq = xr[i + e] * xr[i + e];
                acc[e] = acc[e] + sq;
            }
        float ss = red_add(acc);
        for (; i < dim; i++) ss += xr[i] * xr[i];
        const float inv = 1.0f / sqrtf(ss / (float)dim + c->eps);
        float *o = c->out + r * dim;
        for (i = 0; i < dim; i++) {
            const float t = xr[i] * inv;
            o[i] = t * c->scale[i];
        }
    }
}

void orc_rms_norm(size_t threads, float *out, const float *x, size_t rows, size_t dim, const float *scale,
                  float eps) {
    const norm_ctx c = {out, x, dim, scale, eps};
    orc_for_range_min(threads, rows, 64, &c, rms_norm_rows);
}

/* nn.relu (src/core/nn.zig:436-444). */
void orc_relu(float *x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = x[i] > 0.f ? x[i] : 0.f;
}

/* Model.encode's layer loop and final norm (src/chronos2/model.zig:144-206): per layer, time
 * attention (timeAttention, :208-262: q/k/v linear, the serial RoPE loop, TimeJob over
 * (series, head) with Mask.pick(false, keys_all_valid, true), the o linear), group attention with
 * singleton groups (groupAttention, :264-269: v linear then o linear) and the ReLU MLP, each
 * behind an rmsNorm and added back to x; then the final rmsNorm in place. The attention scale is
 * a parameter here (the model's TimeJob passes 1.0, :306). */
void orc_chronos2_encode(size_t threads, float *x, const uint8_t *key_valid, size_t b, size_t seq, size_t d,
                         size_t nh, size_t hd, size_t d_ff, size_t n_layers, const orc_chronos2_layer *layers,
                         const float *final_norm, float eps, const float *cos_t, const float *sin_t, float scale) {
    const size_t rows = b * seq;
    float *xn = (float *)malloc(rows * d * sizeof(float));
    float *delta = (float *)malloc(rows * d * sizeof(float));
    float *mlp_h = (float *)malloc(rows * d_ff * sizeof(float));
    float *qb = (float *)malloc(rows * d * sizeof(float));
    float *kb = (float *)malloc(rows * d * sizeof(float));
    float *vb = (float *)malloc(rows * d * sizeof(float));
    float *ab = (float *)malloc(rows * d * sizeof(float));
    int all_valid = 1;
    for (size_t i = 0; i < rows; i++) all_valid = all_valid && key_valid[i] != 0;
    for (size_t l = 0; l < n_layers; l++) {
        const orc_chronos2_layer *ly = &layers[l];
        orc_rms_norm(threads, xn, x, rows, d, ly->time_norm, eps);
        orc_linear(threads, qb, xn, rows, ly->time_q, d, d, NULL);
        orc_linear(threads, kb, xn, rows, ly->time_k, d, d, NULL);
        orc_linear(threads, vb, xn, rows, ly->time_v, d, d, NULL);
        orc_chronos2_rope(qb, kb, cos_t, sin_t, rows, seq, d, nh, hd);
        orc_chronos2_time_attention(threads, qb, kb, vb, ab, key_valid, all_valid, b, seq, d, nh, hd, scale);
        orc_linear(threads, delta, ab, rows, ly->time_o, d, d, NULL);
        orc_add_in_place(x, delta, rows * d);

        orc_rms_norm(threads, xn, x, rows, d, ly->group_norm, eps);
        orc_linear(threads, vb, xn, rows, ly->group_v, d, d, NULL);
        orc_linear(threads, delta, vb, rows, ly->group_o, d, d, NULL);
        orc_add_in_place(x, delta, rows * d);

        orc_rms_norm(threads, xn, x, rows, d, ly->mlp_norm, eps);
        orc_linear(threads, mlp_h, xn, rows, ly->mlp_wi, d_ff, d, NULL);
        orc_relu(mlp_h, rows * d_ff);
        orc_linear(threads, delta, mlp_h, rows, ly->mlp_wo, d, d_ff, NULL);
        orc_add_in_place(x, delta, rows * d);
    }
    orc_rms_norm(threads, x, x, rows, d, final_norm, eps);
    free(xn); free(delta); free(mlp_h); free(qb); free(kb); free(vb); free(ab);
}

/* ResBlock(.relu).forward (src/core/resblock.zig:63-79): y = output(relu(hidden(x))) + residual(x),
 * each nn.linear with its bias, the residual added last (addInPlace). */
void orc_resblock_relu(size_t threads, float *y, const float *x, size_t rows, const orc_resblock *rb) {
    const size_t in = rb->in, hid = rb->hid, out = rb->out;
    float *h = (float *)malloc(rows * hid * sizeof(float));
    float *r = (float *)malloc(rows * out * sizeof(float));
    orc_linear(threads, h, x, rows, rb->hidden_w, hid, in, rb->hidden_b);
    orc_relu(h, rows * hid);
    orc_linear(threads, y, h, rows, rb->output_w, out, hid, rb->output_b);
    orc_linear(threads, r, x, rows, rb->residual_w, out, in, rb->residual_b);
    orc_add_in_place(y, r, rows * out);
    free(h);
    free(r);
}

/* The model part of the Chronos-2 forecaster's runChunk (src/chronos2/forecaster.zig:155-183):
 * embed the context and future patch features, lay out [context; REG; future] with its key
 * validity, encode, take the future tokens' hidden states and run the output head. raw:
 * (b * n_out, output_embed->out). */
void orc_chronos2_model_forward(size_t threads, float *raw, const float *feats, const float *fut_feats,
                                const uint8_t *ctx_valid, const float *reg, size_t b, size_t n_ctx, size_t n_out,
                                size_t d, size_t nh, size_t hd, size_t d_ff, size_t n_layers,
                                const orc_chronos2_layer *layers, const float *final_norm, float eps,
                                const float *cos_t, const float *sin_t, float scale, const orc_resblock *input_embed,
                                const orc_resblock *output_embed) {
    const size_t seq = n_ctx + 1 + n_out;
    float *emb = (float *)malloc(b * n_ctx * d * sizeof(float) + 1);
    float *fut_emb = (float *)malloc(b * n_out * d * sizeof(float) + 1);
    orc_resblock_relu(threads, emb, feats, b * n_ctx, input_embed);
    orc_resblock_relu(threads, fut_emb, fut_feats, b * n_out, input_embed);
    float *x = (float *)malloc(b * seq * d * sizeof(float));
    uint8_t *kv = (uint8_t *)malloc(b * seq);
    for (size_t li = 0; li < b; li++) {
        const size_t xb = li * seq * d;
        memcpy(x + xb, emb + li * n_ctx * d, n_ctx * d * sizeof(float));
        memcpy(x + xb + n_ctx * d, reg, d * sizeof(float));
        memcpy(x + xb + (n_ctx + 1) * d, fut_emb + li * n_out * d, n_out * d * sizeof(float));
        for (size_t t = 0; t < n_ctx; t++) kv[li * seq + t] = ctx_valid[li * n_ctx + t] != 0;
        kv[li * seq + n_ctx] = 1;
        for (size_t t = 0; t < n_out; t++) kv[li * seq + n_ctx + 1 + t] = 1;
    }
    orc_chronos2_encode(threads, x, kv, b, seq, d, nh, hd, d_ff, n_layers, layers, final_norm, eps, cos_t, sin_t,
                        scale);
    float *hidden = (float *)malloc(b * n_out * d * sizeof(float) + 1);
    for (size_t li = 0; li < b; li++)
        memcpy(hidden + li * n_out * d, x + (li * seq + n_ctx + 1) * d, n_out * d * sizeof(float));
    orc_resblock_relu(threads, raw, hidden, b * n_out, output_embed);
    free(emb); free(fut_emb); free(x); free(kv); free(hidden);
}

/* The model part of the Chronos-Bolt forecaster's chunk (src/chronos_bolt/forecaster.zig:199-213):
 * embed the patch features, [patches; REG] with its key validity, Model.encode
 * (src/chronos_bolt/model.zig:210-254), Model.decode (:258-308), the output head. */
void orc_bolt_model_forward(size_t threads, float *raw, const float *feats, const uint8_t *patch_valid,
                            const float *reg, const float *dec_start, const float *rel_table, uint32_t num_buckets,
                            uint32_t max_distance, size_t b, size_t n_patch, size_t d, size_t nh, size_t hd,
                            size_t d_ff, const orc_bolt_enc_layer *enc, size_t n_enc, const float *enc_final_norm,
                            const orc_bolt_dec_layer *dec, size_t n_dec, const float *dec_final_norm, float eps,
                            const orc_resblock *input_embed, const orc_resblock *output_embed) {
    const size_t seq = n_patch + 1, rows = b * seq, inner = nh * hd;
    float *emb = (float *)malloc(b * n_patch * d * sizeof(float) + 1);
    orc_resblock_relu(threads, emb, feats, b * n_patch, input_embed);
    float *x = (float *)malloc(rows * d * sizeof(float));
    uint8_t *kv = (uint8_t *)malloc(rows);
    int all_valid = 1;
    for (size_t li = 0; li < b; li++) {
        memcpy(x + li * seq * d, emb + li * n_patch * d, n_patch * d * sizeof(float));
        memcpy(x + (li * seq + n_patch) * d, reg, d * sizeof(float));
        for (size_t p = 0; p < n_patch; p++) {
            kv[li * seq + p] = patch_valid[li * n_patch + p] != 0;
            all_valid = all_valid && kv[li * seq + p];
        }
        kv[li * seq + n_patch] = 1;
    }
    float *xn = (float *)malloc(rows * d * sizeof(float));
    float *delta = (float *)malloc(rows * d * sizeof(float));
    float *h = (float *)malloc(rows * d_ff * sizeof(float));
    float *qb = (float *)malloc(rows * inner * sizeof(float));
    float *kb = (float *)malloc(rows * inner * sizeof(float));
    float *vb = (float *)malloc(rows * inner * sizeof(float));
    float *ab = (float *)malloc(rows * inner * sizeof(float));
    float *bias = (float *)malloc(nh * seq * seq * sizeof(float));
    orc_position_bias(bias, rel_table, seq, nh, num_buckets, max_distance);
    for (size_t l = 0; l < n_enc; l++) {
        const orc_bolt_enc_layer *ly = &enc[l];
        orc_rms_norm(threads, xn, x, rows, d, ly->attn_norm, eps);
        orc_linear(threads, qb, xn, rows, ly->q, inner, d, NULL);
        orc_linear(threads, kb, xn, rows, ly->k, inner, d, NULL);
        orc_linear(threads, vb, xn, rows, ly->v, inner, d, NULL);
        orc_bolt_self_attention(threads, qb, kb, vb, ab, bias, kv, all_valid, b, seq, inner, nh, hd);
        orc_linear(threads, delta, ab, rows, ly->o, d, inner, NULL);
        orc_add_in_place(x, delta, rows * d);
        orc_rms_norm(threads, xn, x, rows, d, ly->ffn_norm, eps);
        orc_linear(threads, h, xn, rows, ly->wi, d_ff, d, NULL);
        orc_relu(h, rows * d_ff);
        orc_linear(threads, delta, h, rows, ly->wo, d, d_ff, NULL);
        orc_add_in_place(x, delta, rows * d);
    }
    orc_rms_norm(threads, x, x, rows, d, enc_final_norm, eps);
    float *y = (float *)malloc(b * d * sizeof(float));
    for (size_t r = 0; r < b; r++) memcpy(y + r * d, dec_start, d * sizeof(float));
    for (size_t l = 0; l < n_dec; l++) {
        const orc_bolt_dec_layer *ly = &dec[l];
        orc_rms_norm(threads, xn, y, b, d, ly->self_norm, eps);
        orc_linear(threads, vb, xn, b, ly->self_v, inner, d, NULL);
        orc_linear(threads, delta, vb, b, ly->self_o, d, inner, NULL);
        orc_add_in_place(y, delta, b * d);
        orc_rms_norm(threads, xn, y, b, d, ly->cross_norm, eps);
        orc_linear(threads, qb, xn, b, ly->cross_q, inner, d, NULL);
        orc_linear(threads, kb, x, rows, ly->cross_k, inner, d, NULL);
        orc_linear(threads, vb, x, rows, ly->cross_v, inner, d, NULL);
        orc_bolt_cross_attention(threads, qb, kb, vb, ab, kv, b, seq, inner, nh, hd);
        orc_linear(threads, delta, ab, b, ly->cross_o, d, inner, NULL);
        orc_add_in_place(y, delta, b * d);
        orc_rms_norm(threads, xn, y, b, d, ly->ffn_norm, eps);
        orc_linear(threads, h, xn, b, ly->wi, d_ff, d, NULL);
        orc_relu(h, b * d_ff);
        orc_linear(threads, delta, h, b, ly->wo, d, d_ff, NULL);
        orc_add_in_place(y, delta, b * d);
    }
    orc_rms_norm(threads, xn, y, b, d, dec_final_norm, eps);
    orc_resblock_relu(threads, raw, xn, b, output_embed);
    free(emb); free(x); free(kv); free(xn); free(delta); free(h); free(qb); free(kb); free(vb); free(ab);
    free(bias); free(y);
}

/* The Chronos-Bolt forecaster's runChunk (src/chronos_bolt/forecaster.zig:130-220) for n series:
 * per series the instance norm over observed values (double sums; a zero scale becomes norm_eps),
 * the [values, mask] patch features left-padded to whole patches and the patch validity, the
 * model forward, and out = raw * scale + loc. out: (n, output_embed->out). */
void orc_bolt_forecast(size_t threads, float *out, const float *ctx, size_t stride, size_t offset, size_t len,
                       size_t n, size_t ps, float norm_eps, const float *reg, const float *dec_start,
                       const float *rel_table, uint32_t num_buckets, uint32_t max_distance, size_t d, size_t nh,
                       size_t hd, size_t d_ff, const orc_bolt_enc_layer *enc, size_t n_enc,
                       const float *enc_final_norm, const orc_bolt_dec_layer *dec, size_t n_dec,
                       const float *dec_final_norm, float eps, const orc_resblock *input_embed,
                       const orc_resblock *output_embed) {
    const size_t pad = (ps - len % ps) % ps, n_patch = (len + pad) / ps, per = output_embed->out;
    float *loc = (float *)malloc(n * sizeof(float)), *scale = (float *)malloc(n * sizeof(float));
    float *feats = (float *)calloc(n * n_patch * 2 * ps + 1, sizeof(float));
    uint8_t *pv = (uint8_t *)calloc(n * n_patch + 1, 1);
    for (size_t li = 0; li < n; li++) {
        const float *row = ctx + li * stride + offset;
        double count = 0, sum = 0;
        for (size_t i = 0; i < len; i++)
            if (!isnan(row[i])) {
                count += 1;
                sum += row[i];
            }
        float lo = 0, sc = 1;
        if (count > 0) {
            lo = (float)(sum / count);
            double ss = 0;
            for (size_t i = 0; i < len; i++)
                if (!isnan(row[i])) {
                    const float dv = row[i] - lo;
                    ss += (double)dv * (double)dv;
                }
            sc = (float)sqrt(ss / count);
            if (sc == 0) sc = norm_eps;
        }
        loc[li] = lo;
        scale[li] = sc;
        for (size_t p = 0; p < n_patch; p++) {
            int any = 0;
            float *f = feats + (li * n_patch + p) * 2 * ps;
            for (size_t i = 0; i < ps; i++) {
                const long src = (long)(p * ps + i) - (long)pad;
                int obs = 0;
                float val = 0;
                if (src >= 0 && !isnan(row[src])) {
                    obs = 1;
                    val = (row[src] - lo) / sc;
                }
                f[i] = val;
                f[ps + i] = obs ? 1.f : 0.f;
                any = any || obs;
            }
            pv[li * n_patch + p] = (uint8_t)any;
        }
    }
    float *raw = (float *)malloc(n * per * sizeof(float));
    orc_bolt_model_forward(threads, raw, feats, pv, reg, dec_start, rel_table, num_buckets, max_distance, n, n_patch, d,
                           nh, hd, d_ff, enc, n_enc, enc_final_norm, dec, n_dec, dec_final_norm, eps, input_embed,
                           output_embed);
    for (size_t li = 0; li < n; li++)
        for (size_t j = 0; j < per; j++) {
            const float t = raw[li * per + j] * scale[li];
            out[li * per + j] = t + loc[li];
        }
    free(loc); free(scale); free(feats); free(pv); free(raw);
}

float orc_quantile_linear(const float *sorted, size_t n, float level) {
    const float rank = level * (float)(n - 1);
    const float lo_f = floorf(rank);
    const size_t lo = (size_t)lo_f;
    size_t hi = (size_t)ceilf(rank);
    if (hi > n - 1) hi = n - 1;
    const float w = rank - lo_f, a = sorted[lo], bb = sorted[hi];
    if (w < 0.5f) {
        const float t = w * (bb - a);
        return a + t;
    }
    const float t = (bb - a) * (1 - w);
    return bb - t;
}

static int orc_cmp_f32(const void *x, const void *y) {
    const float a = *(const float *)x, b = *(const float *)y;
    return a < b ? -1 : (a > b ? 1 : 0);
}

static void orc_bolt_block(size_t threads, float *out, const float *ctx, size_t stride, size_t offset, size_t len,
                           size_t n, size_t ps, float norm_eps, const orc_bolt_model *m) {
    orc_bolt_forecast(threads, out, ctx, stride, offset, len, n, ps, norm_eps, m->reg, m->dec_start, m->rel_table,
                      m->num_buckets, m->max_distance, m->d, m->nh, m->hd, m->d_ff, m->enc, m->n_enc, m->enc_final_norm,
                      m->dec, m->n_dec, m->dec_final_norm, m->eps, m->input_embed, m->output_embed);
}

/* storeBlock (forecaster.zig:95-103): pred (b, q, P) into out (b, horizon, q) from step start. */
static void orc_bolt_store(float *out, const float *pred, size_t b, size_t q, size_t P, size_t horizon, size_t start) {
    for (size_t s = 0; s < b; s++)
        for (size_t p = 0; p < P && start + p < horizon; p++)
            for (size_t qi = 0; qi < q; qi++) out[(s * horizon + start + p) * q + qi] = pred[(s * q + qi) * P + p];
}

void orc_bolt_forecast_horizon(size_t threads, float *out, const float *inputs, size_t b, size_t t_in, size_t horizon,
                               size_t ps, size_t P, size_t max_ctx, const float *levels, size_t q, float norm_eps,
                               const orc_bolt_model *m) {
    const size_t len0 = t_in < max_ctx ? t_in : max_ctx;
    float *pred = (float *)malloc(b * q * P * sizeof(float));
    orc_bolt_block(threads, pred, inputs, t_in, t_in - len0, len0, b, ps, norm_eps, m);
    orc_bolt_store(out, pred, b, q, P, horizon, 0);
    size_t done = P < horizon ? P : horizon;
    if (done < horizon) {
        /* every quantile path its own context row */
        size_t len = len0;
        float *cur = (float *)malloc(b * q * len * sizeof(float));
        for (size_t s = 0; s < b; s++)
            for (size_t qi = 0; qi < q; qi++)
                memcpy(cur + (s * q + qi) * len, inputs + s * t_in + t_in - len0, len0 * sizeof(float));
        float *samples = (float *)malloc(q * q * sizeof(float));
        float *raw = (float *)malloc(b * q * q * P * sizeof(float));
        while (done < horizon) {
            const size_t new_len = len + P < max_ctx ? len + P : max_ctx, skip = len + P - new_len;
            float *next = (float *)malloc(b * q * new_len * sizeof(float));
            for (size_t row = 0; row < b * q; row++)
                for (size_t i = 0; i < new_len; i++) {
                    const size_t j = skip + i;
                    next[row * new_len + i] = j < len ? cur[row * len + j] : pred[row * P + (j - len)];
                }
            free(cur);
            cur = next;
            len = new_len;
            orc_bolt_block(threads, raw, cur, len, 0, len, b * q, ps, norm_eps, m);
            for (size_t s = 0; s < b; s++)
                for (size_t p = 0; p < P; p++) {
                    for (size_t k = 0; k < q * q; k++) samples[k] = raw[(s * q * q + k) * P + p];
                    qsort(samples, q * q, sizeof(float), orc_cmp_f32);
                    for (size_t qi = 0; qi < q; qi++)
                        pred[(s * q + qi) * P + p] = orc_quantile_linear(samples, q * q, levels[qi]);
                }
            orc_bolt_store(out, pred, b, q, P, horizon, done);
            done += P;
        }
        free(cur); free(samples); free(raw);
    }
    free(pred);
}

/* src/chronos2/forecaster.zig:59-204 (runChunk) for the series of one chunk. */
void orc_chronos2_forecast(size_t threads, float *out, const float *inputs, size_t stride, size_t start, size_t len,
                           size_t n, size_t ps, size_t horizon, float time_scale, int arcsinh, const float *reg,
                           size_t d, size_t nh, size_t hd, size_t d_ff, size_t n_layers,
                           const orc_chronos2_layer *layers, const float *final_norm, float eps, const float *cos_t,
                           const float *sin_t, float scale, const orc_resblock *input_embed,
                           const orc_resblock *output_embed) {
    const size_t pad = (ps - len % ps) % ps, n_ctx = (len + pad) / ps, n_out = (horizon + ps - 1) / ps;
    const size_t q = output_embed->out / ps;
    float *loc = (float *)malloc((n + 1) * sizeof(float)), *scl = (float *)malloc((n + 1) * sizeof(float));
    float *feats = (float *)calloc(n * n_ctx * 3 * ps + 1, sizeof(float));
    float *fut = (float *)calloc(n * n_out * 3 * ps + 1, sizeof(float));
    uint8_t *cv = (uint8_t *)calloc(n * n_ctx + 1, 1);
    for (size_t li = 0; li < n; li++) {
        const float *row = inputs + li * stride + start;
        double count = 0, sum = 0;
        for (size_t i = 0; i < len; i++)
            if (!isnan(row[i])) {
                count += 1;
                sum += row[i];
            }
        float lo = 0, sc = 1;
        if (count > 0) {
            lo = (float)(sum / count);
            double ss = 0;
            for (size_t i = 0; i < len; i++)
                if (!isnan(row[i])) {
                    const float dv = row[i] - lo;
                    ss += (double)dv * (double)dv;
                }
            sc = (float)sqrt(ss / count);
            if (sc == 0) sc = 1e-5f;
        }
        loc[li] = lo;
        scl[li] = sc;
        for (size_t p = 0; p < n_ctx; p++) {
            int any = 0;
            float *f = feats + (li * n_ctx + p) * 3 * ps;
            for (size_t i = 0; i < ps; i++) {
                const size_t j = p * ps + i;
                const long src = (long)j - (long)pad;
                int obs = 0;
                float val = 0;
                if (src >= 0 && src < (long)len && !isnan(row[src])) {
                    obs = 1;
                    val = (row[src] - lo) / sc;
                    if (arcsinh) val = asinhf(val);
                }
                f[i] = ((float)j - (float)(n_ctx * ps)) / time_scale;
                f[ps + i] = val;
                f[2 * ps + i] = obs ? 1.f : 0.f;
                any = any || obs;
            }
            cv[li * n_ctx + p] = (uint8_t)any;
        }
        for (size_t p = 0; p < n_out; p++) {
            float *f = fut + (li * n_out + p) * 3 * ps;
            for (size_t i = 0; i < ps; i++) f[i] = (float)(p * ps + i) / time_scale;
        }
    }
    float *raw = (float *)malloc((n * n_out * q * ps + 1) * sizeof(float));
    orc_chronos2_model_forward(threads, raw, feats, fut, cv, reg, n, n_ctx, n_out, d, nh, hd, d_ff, n_layers, layers,
                               final_norm, eps, cos_t, sin_t, scale, input_embed, output_embed);
    for (size_t li = 0; li < n; li++)
        for (size_t p = 0; p < n_out; p++)
            for (size_t i = 0; i < ps; i++) {
                const size_t step = p * ps + i;
                if (step >= horizon) continue;
                for (size_t qi = 0; qi < q; qi++) {
                    float v = raw[(li * n_out + p) * q * ps + qi * ps + i];
                    if (arcsinh) v = sinhf(v);
                    const float t = v * scl[li];
                    out[(li * horizon + step) * q + qi] = t + loc[li];
                }
            }
    free(loc); free(scl); free(feats); free(fut); free(cv); free(raw);
}

/* ------------------------------------------------------------------------------------------ */
/* Timestral (src/timestral/model.zig) */

int orc_timestral_key_valid(uint8_t *key_valid, size_t *first_obs, const uint8_t *obs, size_t rows, size_t vall,
                            size_t ne, size_t ps, int attend_missing) {
    const size_t w = ne * ps, groups = vall ? rows / vall : 0;
    for (size_t g = 0; g < groups; g++) first_obs[g] = ne;
    for (size_t r = 0; r < rows; r++) {
        const size_t g = r / vall;
        int started = 0;
        for (size_t p = 0; p < ne; p++) {
            int ob = 0;
            for (size_t i = 0; i < ps; i++) ob = ob || obs[r * w + p * ps + i] != 0;
            if (ob && p < first_obs[g]) first_obs[g] = p;
            started = started || ob;
            key_valid[r * ne + p] = (uint8_t)(attend_missing ? (ob || started) : ob);
        }
    }
    for (size_t g = 0; g < groups; g++)
        if (first_obs[g] == ne) first_obs[g] = 0;
    int all = 1;
    for (size_t i = 0; i < rows * ne; i++) all = all && key_valid[i];
    return all;
}

void orc_timestral_rope_tables(float *cos_t, float *sin_t, size_t groups, size_t ne, size_t l, size_t h,
                               size_t hd, size_t rope_dim, float theta, const size_t *first_obs) {
    const size_t half = hd / 2, sl = ne + h;
    float *inv_freq = (float *)calloc(half ? half : 1, sizeof(float));
    for (size_t i = 0; i < rope_dim / 2; i++) {
        const float idx = (float)(2 * i);
        inv_freq[i] = 1.0f / powf(theta, idx / (float)rope_dim);
    }
    for (size_t g = 0; g < groups; g++)
        for (size_t tok = 0; tok < sl; tok++) {
            const int64_t time = tok < ne ? (int64_t)tok : (int64_t)(l + tok - ne);
            const float pos = (float)(time - (int64_t)first_obs[g]);
            for (size_t i = 0; i < half; i++) {
                const float ang = inv_freq[i] * pos;
                cos_t[(g * sl + tok) * half + i] = cosf(ang);
                sin_t[(g * sl + tok) * half + i] = sinf(ang);
            }
        }
    free(inv_freq);
}

typedef struct {
    float *qkv;
    const float *cos_t, *sin_t;
    size_t sl, vall, d, nh, hd;
} ts_rope_job;

static void ts_rope(const void *p, size_t t0, size_t t1) {
    const ts_rope_job *j = (const ts_rope_job *)p;
    const size_t half = j->hd / 2, d = j->d;
    for (size_t idx = t0; idx < t1; idx++) {
        const size_t r = idx / j->sl, tok = idx % j->sl, g = r / j->vall;
        const float *cs = j->cos_t + (g * j->sl + tok) * half, *sn = j->sin_t + (g * j->sl + tok) * half;
        const size_t base = idx * 3 * d;
        for (size_t hh = 0; hh < j->nh; hh++) {
            orc_rope_half(j->qkv + base + hh * j->hd, cs, sn, half);
            orc_rope_half(j->qkv + base + d + hh * j->hd, cs, sn, half);
        }
    }
}

void orc_timestral_rope(size_t threads, float *qkv, const float *cos_t, const float *sin_t, size_t rows,
                        size_t sl, size_t vall, size_t d, size_t nh, size_t hd) {
    const ts_rope_job job = {qkv, cos_t, sin_t, sl, vall, d, nh, hd};
    orc_for_range_min(threads, rows * sl, 16, &job, ts_rope);
}

typedef struct {
    const float *qkv;
    float *o;
    const uint8_t *key_valid;
    int keys_all_valid;
    const uint8_t *bidir;
    size_t ne, l, h, d, nh, hd;
} ts_time_job;

static void ts_time_attend(const void *p, size_t first, size_t last) {
    const ts_time_job *j = (const ts_time_job *)p;
    const size_t d = j->d, nh = j->nh, hd = j->hd, ne = j->ne, l = j->l, h = j->h, sl = ne + h;
    const float sm_scale = 1.0f / sqrtf((float)hd);
    const float ninf = -INFINITY;
    const size_t cap = ne * ne > h * sl ? ne * ne : h * sl;
    float *scores = (float *)malloc((cap ? cap : 1) * sizeof(float));
    const size_t st[4] = {3 * d, 3 * d, 3 * d, d};
    for (size_t item = first; item < last; item++) {
        const size_t r = item / nh, hh = item % nh, off = hh * hd;
        const int bidir = j->bidir ? j->bidir[r] != 0 : 0;
        const size_t base = r * sl * 3 * d;
        const float *q = j->qkv + base + off;
        const float *k = j->qkv + base + d + off;
        const float *v = j->qkv + base + 2 * d + off;
        float *o = j->o + r * sl * d + off;
        const uint8_t *kv = j->key_valid + r * ne;

        const int mask = orc_mask_pick(!bidir, j->keys_all_valid, 0);
        orc_self_attend(mask, scores, q, k, v, o, st, ne, hd, sm_scale, kv, NULL);
        orc_gemm_nt(scores, sl, j->qkv + base + ne * 3 * d + off, 3 * d, k, 3 * d, h, sl, hd, sm_scale);
        if (j->keys_all_valid) {
            for (size_t jj = 0; jj < h; jj++) {
                float *row = scores + jj * sl;
                for (size_t kk = l; kk < ne; kk++) row[kk] = ninf;
                const size_t end = ne + jj + 1;
                orc_softmax(row, end);
                for (size_t kk = end; kk < sl; kk++) row[kk] = 0;
            }
        } else {
            for (size_t jj = 0; jj < h; jj++) {
                float *row = scores + jj * sl;
                for (size_t kk = 0; kk < ne; kk++)
                    if (kk >= l || !kv[kk]) row[kk] = ninf;
                for (size_t kk = ne + jj + 1; kk < sl; kk++) row[kk] = ninf;
                orc_softmax(row, sl);
            }
        }
        orc_gemm_nn(o + ne * d, d, scores, sl, v, 3 * d, h, hd, sl);
    }
    free(scores);
}

void orc_timestral_time_attention(size_t threads, const float *qkv, float *o, const uint8_t *key_valid,
                                  int keys_all_valid, const uint8_t *bidir, size_t rows, size_t ne,
                                  size_t l, size_t h, size_t d, size_t nh, size_t hd) {
    const ts_time_job job = {qkv, o, key_valid, keys_all_valid, bidir, ne, l, h, d, nh, hd};
    orc_for_range_min(threads, rows * nh, 1, &job, ts_time_attend);
}

/* ------------------------------------------------------------------------------------------ */
/* Timestral variate attention, VariateJob.run (src/timestral/model.zig:648-709): at every
 * (series group, token slot) the vall rows of the group attend each other, per head. The allowed
 * matrix is built once per item: the diagonal is always open; another row is read on an encoder
 * slot only if its patch is a valid key; with covariates, a non-target row never reads a target
 * row and a known-future row never reads a non-known row. Scores nn.dot(q, k) * 1/sqrt(hd),
 * nn.softmax, then o = sum of w * v over the rows with w != 0, in row order (mulAddInPlace). */

typedef struct {
    const float *qkv;
    float *o;
    const uint8_t *key_valid;
    const uint8_t *roles;
    int cov;
    size_t vall, ne, sl, d, nh, hd;
} ts_variate_job;

enum { ORC_ROLE_TARGET = 0, ORC_ROLE_PAST = 1, ORC_ROLE_KNOWN = 2 }; /* model.zig:89 order */

static void ts_variate_run(const void *p, size_t first, size_t last) {
    const ts_variate_job *j = (const ts_variate_job *)p;
    const size_t vall = j->vall, ne = j->ne, sl = j->sl, d = j->d, nh = j->nh, hd = j->hd;
    const float sm_scale = 1.0f / sqrtf((float)hd);
    const float ninf = -INFINITY;
    float *sc = (float *)malloc(vall * sizeof(float));
    uint8_t *allowed = (uint8_t *)malloc(vall * vall);
    for (size_t item = first; item < last; item++) {
        const size_t g = item / sl, tok = item % sl, r0 = g * vall;
        for (size_t iq = 0; iq < vall; iq++)
            for (size_t ik = 0; ik < vall; ik++) {
                int ok = ik == iq;
                if (!ok) {
                    const int valid = tok >= ne || j->key_valid[(r0 + ik) * ne + tok];
                    int forbidden = 0;
                    if (j->cov) {
                        const int rq = j->roles[iq], rk = j->roles[ik];
                        forbidden = (rq != ORC_ROLE_TARGET && rk == ORC_ROLE_TARGET) ||
                                    (rq == ORC_ROLE_KNOWN && rk != ORC_ROLE_KNOWN);
                    }
                    ok = valid && !forbidden;
                }
                allowed[iq * vall + ik] = (uint8_t)ok;
            }
        for (size_t hh = 0; hh < nh; hh++) {
            const size_t qoff = hh * hd;
            for (size_t iq = 0; iq < vall; iq++) {
                const float *qsrc = j->qkv + (r0 + iq) * sl * 3 * d + tok * 3 * d + qoff;
                for (size_t ik = 0; ik < vall; ik++) {
                    if (!allowed[iq * vall + ik]) {
                        sc[ik] = ninf;
                        continue;
                    }
                    const float *ksrc = j->qkv + (r0 + ik) * sl * 3 * d + tok * 3 * d + d + qoff;
                    sc[ik] = orc_dot(qsrc, ksrc, hd) * sm_scale;
                }
                orc_softmax(sc, vall);
                float *dst = j->o + (r0 + iq) * sl * d + tok * d + qoff;
                memset(dst, 0, hd * sizeof(float));
                for (size_t ik = 0; ik < vall; ik++) {
                    const float w = sc[ik];
                    if (w == 0) continue;
                    orc_mul_add_in_place(dst, j->qkv + (r0 + ik) * sl * 3 * d + tok * 3 * d + 2 * d + qoff, hd, w);
                }
            }
        }
    }
    free(allowed);
    free(sc);
}

void orc_timestral_variate_attention(size_t threads, const float *qkv, float *o, const uint8_t *key_valid,
                                     const uint8_t *roles, int cov, size_t groups, size_t vall, size_t ne,
                                     size_t h, size_t d, size_t nh, size_t hd) {
    const ts_variate_job job = {qkv, o, key_valid, roles, cov, vall, ne, ne + h, d, nh, hd};
    orc_for_range_min(threads, groups * (ne + h), 8, &job, ts_variate_run);
}

/* nn.mulSigmoid (src/core/nn.zig:423-433): dst = x / (1 + expVec(-g)) over whole vectors (unfused
 * division), x * sigmoid(g) = x * (1 / (1 + @exp(-g))) over the tail. */
void orc_mul_sigmoid(float *dst, const float *x, const float *g, size_t n) {
    size_t i = 0;
    for (; i + L <= n; i += L)
        for (int e = 0; e < L; e++) dst[i + e] = x[i + e] / (1.0f + orc_exp_vec(-g[i + e]));
    for (; i < n; i++) dst[i] = x[i] * (1.0f / (1.0f + expf(-g[i])));
}

/* ------------------------------------------------------------------------------------------ */
/* Generic batched selfAttend. */

typedef struct {
    int mask;
    const float *q, *k, *v;
    float *o;
    size_t q_tok, q_batch, k_tok, k_batch, v_tok, v_batch, o_tok, o_batch;
    const uint8_t *key_valid;
    size_t kv_batch;
    const float *bias;
    size_t nh, n, hd;
    float scale;
} batched_job;

static void batched_attend(const void *p, size_t first, size_t last) {
    const batched_job *j = (const batched_job *)p;
    const size_t n = j->n, hd = j->hd;
    float *scores = (float *)malloc((n > 0 ? n * n : 1) * sizeof(float));
    const size_t st[4] = {j->q_tok, j->k_tok, j->v_tok, j->o_tok};
    for (size_t item = first; item < last; item++) {
        const size_t b = item / j->nh, h = item % j->nh;
        orc_self_attend(j->mask, scores, j->q + b * j->q_batch + h * hd, j->k + b * j->k_batch + h * hd,
                        j->v + b * j->v_batch + h * hd, j->o + b * j->o_batch + h * hd, st, n, hd, j->scale,
                        j->key_valid ? j->key_valid + b * j->kv_batch : NULL,
                        j->bias ? j->bias + h * n * n : NULL);
    }
    free(scores);
}

void orc_batched_self_attend(size_t threads, int mask, const float *q, size_t q_tok, size_t q_batch,
                             const float *k, size_t k_tok, size_t k_batch, const float *v, size_t v_tok,
                             size_t v_batch, float *o, size_t o_tok, size_t o_batch,
                             const uint8_t *key_valid, size_t kv_batch, const float *bias,
                             size_t nb, size_t nh, size_t n, size_t hd, float scale) {
    const batched_job job = {mask,    q,       k,       v,         o,        q_tok, q_batch, k_tok,
                             k_batch, v_tok,   v_batch, o_tok,     o_batch,  key_valid, kv_batch,
                             bias,    nh,      n,       hd,        scale};
    orc_for_range_min(threads, nb * nh, 1, &job, batched_attend);
}
