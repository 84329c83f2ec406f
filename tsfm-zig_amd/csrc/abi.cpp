// extern "C" ABI of libtsfm_attn.so (declared in include/tsfm_attn.h).
//
// Mirrors the reference backend's conventions (src/platform/cuda/gemm.c): one-time device set-up
// under pthread_once (:112-166), one stream and growable device staging buffer per host thread
// kept in a pthread key with a destructor (:171-227), synchronous host round trip for host
// pointers (:252-314), int return with 0 = success and anything else = "use the CPU" (:1-15).
// Unlike the reference, a call covers a whole batch of (series, head) items and the device work
// is one fused kernel instead of two cuBLAS GEMMs per item.
#include <hip/hip_runtime.h>
#include <pthread.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/tsfm_attn.h"
#include "abi_internal.hpp"
#include "launch.hpp"

namespace tsfm {
namespace abi {

pthread_once_t g_once = PTHREAD_ONCE_INIT;
int g_ready = 0;
int g_device = 0;
char g_init_err[256] = "not initialised";
thread_local char t_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof t_err, fmt, ap);
    va_end(ap);
    return code;
}

void init_once() {
    const char* dis = getenv("TSFM_HIP_DISABLE");
    if (dis != nullptr && dis[0] != '\0' && strcmp(dis, "0") != 0) {
        snprintf(g_init_err, sizeof g_init_err, "disabled by TSFM_HIP_DISABLE");
        return;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        snprintf(g_init_err, sizeof g_init_err, "no HIP device");
        fprintf(stderr, "tsfm_attn unavailable: %s\n", g_init_err);
        return;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        snprintf(g_init_err, sizeof g_init_err, "cannot query device %d", dev);
        fprintf(stderr, "tsfm_attn unavailable: %s\n", g_init_err);
        return;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        snprintf(g_init_err, sizeof g_init_err, "device %d is %s, the kernels are built for gfx950", dev,
                 prop.gcnArchName);
        fprintf(stderr, "tsfm_attn unavailable: %s\n", g_init_err);
        return;
    }
    g_device = dev;
    g_ready = 1;
}

int ensure_ready() {
    pthread_once(&g_once, init_once);
    if (!g_ready) return fail(TSFM_E_UNAVAILABLE, "%s", g_init_err);
    return TSFM_OK;
}

int hip_fail(hipError_t e, const char* what) {
    if (e == hipErrorNotSupported) return fail(TSFM_E_UNSUPPORTED, "%s: not supported", what);
    return fail(TSFM_E_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace abi
}  // namespace tsfm

using tsfm::abi::ensure_ready;
using tsfm::abi::fail;
using tsfm::abi::g_device;
using tsfm::abi::hip_fail;
using tsfm::abi::Plan;
using tsfm::abi::t_err;

namespace {

// ---- per-thread stream and staging buffer -------------------------------------------------------

struct ThreadCtx {
    hipStream_t stream = nullptr;
    void* buf = nullptr;
    size_t cap = 0;
    // Split-partials buffers of this thread's device-pointer projections, one per (device, caller
    // stream). Per thread, so that two threads queuing on one stream (the null stream,
    // hipStreamPerThread) never share a buffer between a product and its reduce.
    struct SplitBuf {
        int device;
        hipStream_t stream;
        float* buf;
    };
    std::vector<SplitBuf> splits;
    // Scratch buffers of this thread's device-pointer entry points (scratch_acquire), one per
    // (device, caller stream, entry point).
    struct ScratchBuf {
        int device;
        hipStream_t stream;
        int slot;
        char* buf;
        size_t cap;
    };
    std::vector<ScratchBuf> scratch;
};

constexpr size_t kMaxSplitBufs = 8;  // per thread; more streams take a stream-ordered buffer per call

pthread_key_t g_ctx_key;
pthread_once_t g_ctx_once = PTHREAD_ONCE_INIT;

void destroy_ctx(void* ptr) {
    ThreadCtx* c = static_cast<ThreadCtx*>(ptr);
    if (c == nullptr) return;
    if (c->stream != nullptr) (void)hipStreamDestroy(c->stream);
    if (c->buf != nullptr) (void)hipFree(c->buf);
    // hipFree waits for the device's queued work, so a product still queued on a caller's stream
    // has finished with its partials before they are released.
    for (const ThreadCtx::SplitBuf& b : c->splits) {
        (void)hipSetDevice(b.device);
        (void)hipFree(b.buf);
    }
    for (const ThreadCtx::ScratchBuf& b : c->scratch) {
        (void)hipSetDevice(b.device);
        (void)hipFree(b.buf);
    }
    delete c;
}

void create_ctx_key() { pthread_key_create(&g_ctx_key, destroy_ctx); }

ThreadCtx* thread_ctx() {
    pthread_once(&g_ctx_once, create_ctx_key);
    ThreadCtx* c = static_cast<ThreadCtx*>(pthread_getspecific(g_ctx_key));
    if (c != nullptr) return c;
    c = new ThreadCtx();
    if (hipSetDevice(g_device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        destroy_ctx(c);
        return nullptr;
    }
    pthread_setspecific(g_ctx_key, c);
    return c;
}

int ensure_buf(ThreadCtx* c, size_t bytes) {
    if (c->cap >= bytes) return TSFM_OK;
    void* next = nullptr;
    if (hipMalloc(&next, bytes) != hipSuccess || next == nullptr)
        return fail(TSFM_E_DEVICE, "device staging allocation of %zu bytes failed", bytes);
    if (c->buf != nullptr) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(c->buf);
    }
    c->buf = next;
    c->cap = bytes;
    return TSFM_OK;
}

// The split-partials buffer for a device-pointer projection queued on `stream` by this thread:
// the thread's kept buffer for (device, stream), made on first use; past kMaxSplitBufs streams, a
// stream-ordered allocation that the caller releases with hipFreeAsync after queuing (*owned).
hipError_t split_buf_for(ThreadCtx* c, hipStream_t stream, float** out, bool* owned) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    *owned = false;
    for (const ThreadCtx::SplitBuf& b : c->splits)
        if (b.device == device && b.stream == stream) {
            *out = b.buf;
            return hipSuccess;
        }
    void* buf = nullptr;
    if (c->splits.size() >= kMaxSplitBufs) {
        if ((e = hipMallocAsync(&buf, tsfm::kSplitWorkspaceBytes, stream)) != hipSuccess) return e;
        *owned = true;
    } else {
        if ((e = hipMalloc(&buf, tsfm::kSplitWorkspaceBytes)) != hipSuccess) return e;
        c->splits.push_back({device, stream, static_cast<float*>(buf)});
    }
    *out = static_cast<float*>(buf);
    return hipSuccess;
}

constexpr size_t kMaxScratchBufs = 16;  // per thread; more take a stream-ordered allocation per call

}  // namespace

namespace tsfm {
namespace abi {

// Scratch for an entry point's device work queued on `stream` by this thread: a buffer kept per
// (device, stream, slot) and grown as needed (slot: one per entry point, so that nested calls
// never share one), so that a caller that repeats a call does not pay a stream-ordered allocation
// and release each time (about 30 us of host time per pair). Stream order makes reuse by the
// thread's next call on the same stream safe; another thread has buffers of its own. Growing waits
// for the stream, then replaces the buffer. Past kMaxScratchBufs buffers (or without a thread
// context) it returns a stream-ordered allocation that the caller releases with hipFreeAsync after
// queuing (*owned).
hipError_t scratch_acquire(hipStream_t stream, int slot, size_t bytes, char** out, bool* owned) {
    *owned = false;
    *out = nullptr;
    bytes = std::max<size_t>(bytes, 256);
    ThreadCtx* c = thread_ctx();
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (c != nullptr) {
        for (ThreadCtx::ScratchBuf& b : c->scratch)
            if (b.device == device && b.stream == stream && b.slot == slot) {
                if (b.cap < bytes) {
                    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
                    (void)hipFree(b.buf);
                    b.buf = nullptr;
                    b.cap = 0;
                    void* next = nullptr;
                    if ((e = hipMalloc(&next, bytes)) != hipSuccess) return e;
                    b.buf = static_cast<char*>(next);
                    b.cap = bytes;
                }
                *out = b.buf;
                return hipSuccess;
            }
        if (c->scratch.size() < kMaxScratchBufs) {
            void* buf = nullptr;
            if ((e = hipMalloc(&buf, bytes)) != hipSuccess) return e;
            c->scratch.push_back({device, stream, slot, static_cast<char*>(buf), bytes});
            *out = static_cast<char*>(buf);
            return hipSuccess;
        }
    }
    void* buf = nullptr;
    if ((e = hipMallocAsync(&buf, bytes, stream)) != hipSuccess) return e;
    *out = static_cast<char*>(buf);
    *owned = true;
    return hipSuccess;
}


int run_host_io(std::initializer_list<HostArray> ins, std::initializer_list<HostArray> outs,
                const std::function<int(hipStream_t)>& body) {
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    const hipStream_t s = ctx->stream;
    Plan plan;
    std::vector<size_t> at;
    for (const HostArray& a : ins) at.push_back(plan.take(a.bytes));
    for (const HostArray& a : outs) at.push_back(plan.take(a.bytes));
    char* buf = nullptr;
    hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&buf), plan.off > 0 ? plan.off : 256, s);
    if (e != hipSuccess) return hip_fail(e, "host I/O staging allocation");
    size_t i = 0;
    for (const HostArray& a : ins) {
        *a.dev = a.host != nullptr ? buf + at[i] : nullptr;
        if (e == hipSuccess && a.host != nullptr && a.bytes > 0)
            e = hipMemcpyAsync(buf + at[i], a.host, a.bytes, hipMemcpyHostToDevice, s);
        i++;
    }
    for (const HostArray& a : outs) *a.dev = buf + at[i++];
    if (e == hipSuccess) rc = body(s);
    i = ins.size();
    for (const HostArray& a : outs) {
        if (e == hipSuccess && rc == TSFM_OK && a.bytes > 0)
            e = hipMemcpyAsync(const_cast<void*>(a.host), buf + at[i], a.bytes, hipMemcpyDeviceToHost, s);
        i++;
    }
    const hipError_t f = hipFreeAsync(buf, s);
    const hipError_t y = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "host I/O copy");
    if (rc != TSFM_OK) return rc;
    if (f != hipSuccess) return hip_fail(f, "host I/O staging release");
    if (y != hipSuccess) return hip_fail(y, "stream synchronise");
    return TSFM_OK;
}

}  // namespace abi
}  // namespace tsfm

namespace {


size_t elem_size(int dtype) { return dtype == TSFM_DTYPE_F32 ? 4 : 2; }

// Elements spanned by a (B, n, H*D) view with the given strides.
int64_t span(int64_t B, int64_t n, int64_t tok, int64_t batch, int64_t row) {
    return (B - 1) * batch + (n - 1) * tok + row;
}

// Copy `rows` rows of `width` bytes, pitch `pitch` bytes, per batch, from device to host. Only the
// row contents move: padding between rows (other heads, fused-projection gaps) is left alone.
hipError_t copy_rows_d2h(void* dst, const void* src, int64_t B, int64_t rows, int64_t batch_bytes, int64_t pitch,
                         int64_t width, hipStream_t s) {
    if (batch_bytes == rows * pitch)
        return hipMemcpy2DAsync(dst, pitch, src, pitch, width, B * rows, hipMemcpyDeviceToHost, s);
    for (int64_t b = 0; b < B; b++) {
        hipError_t e = hipMemcpy2DAsync(static_cast<char*>(dst) + b * batch_bytes, pitch,
                                        static_cast<const char*>(src) + b * batch_bytes, pitch, width, rows,
                                        hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Largest element span a strided view may have: 2^46 elements (256 TiB of f32) is past any device or
// host buffer, and keeps every offset sum below it free of int64 overflow.
constexpr int64_t kMaxSpan = (int64_t)1 << 46;

// Elements spanned by a (B, n, row) view with non-negative strides, or -1 when that passes
// kMaxSpan (checked step by step, so no intermediate product overflows).
int64_t span_checked(int64_t B, int64_t n, int64_t tok, int64_t batch, int64_t row) {
    if (B <= 0 || n <= 0) return 0;
    int64_t t1 = 0, t2 = 0, s = 0;
    if (__builtin_mul_overflow(B - 1, batch, &t1) || __builtin_mul_overflow(n - 1, tok, &t2) ||
        __builtin_add_overflow(t1, t2, &s) || __builtin_add_overflow(s, row, &s) || s > kMaxSpan)
        return -1;
    return s;
}

int validate(const tsfm_attn_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (a->dtype < TSFM_DTYPE_F32 || a->dtype > TSFM_DTYPE_F16) return fail(TSFM_E_INVALID, "bad dtype %d", a->dtype);
    if (a->mask < TSFM_MASK_FULL || a->mask > TSFM_MASK_DECODER) return fail(TSFM_E_INVALID, "bad mask %d", a->mask);
    if (a->batch < 0 || a->heads < 0 || a->n_q < 0 || a->n_k < 0) return fail(TSFM_E_INVALID, "negative size");
    if (a->head_dim != 64) return fail(TSFM_E_UNSUPPORTED, "head_dim %d (supported: 64)", a->head_dim);
    if (a->q == nullptr || a->k == nullptr || a->v == nullptr || a->o == nullptr)
        return fail(TSFM_E_INVALID, "q, k, v and o are required");
    if (a->q_tok < 0 || a->q_batch < 0 || a->k_tok < 0 || a->k_batch < 0 || a->v_tok < 0 || a->v_batch < 0 ||
        a->o_tok < 0 || a->o_batch < 0)
        return fail(TSFM_E_INVALID, "negative stride");
    const int64_t vec = a->dtype == TSFM_DTYPE_F32 ? 4 : 8;  // elements per 16-byte load
    if (a->q_tok % vec || a->q_batch % vec || a->k_tok % vec || a->k_batch % vec || a->v_tok % vec ||
        a->v_batch % vec || a->o_tok % vec || a->o_batch % vec)
        return fail(TSFM_E_UNSUPPORTED, "strides must be multiples of 16 bytes");
    const int64_t row = (int64_t)a->heads * a->head_dim;
    if (a->o_tok < row && a->n_q > 1) return fail(TSFM_E_INVALID, "o token stride smaller than heads * head_dim");
    // The kernels address the K and V rows of one (series, head), and the rows of a tile past the
    // last key, through 32-bit byte offsets.
    if (a->dtype != TSFM_DTYPE_F32 && !(a->scale >= 0.f))
        return fail(TSFM_E_UNSUPPORTED, "half-precision attention needs a non-negative scale");
    const int64_t esz = a->dtype == TSFM_DTYPE_F32 ? 4 : 2;
    if (std::max(a->k_tok, a->v_tok) > (0xffffffffLL - 256) / esz / ((int64_t)a->n_k + 64))
        return fail(TSFM_E_UNSUPPORTED, "the K/V rows of one series must span less than 4 GiB");
    if (span_checked(a->batch, a->n_q, a->q_tok, a->q_batch, row) < 0 ||
        span_checked(a->batch, a->n_k, a->k_tok, a->k_batch, row) < 0 ||
        span_checked(a->batch, a->n_k, a->v_tok, a->v_batch, row) < 0 ||
        span_checked(a->batch, a->n_q, a->o_tok, a->o_batch, row) < 0)
        return fail(TSFM_E_UNSUPPORTED, "a q/k/v/o view spans more than 2^46 elements");
    const bool reads_valid = a->mask == TSFM_MASK_KEYS_ADDITIVE || a->mask == TSFM_MASK_CAUSAL_KEYS ||
                             a->mask == TSFM_MASK_FULL_KEYS || a->mask == TSFM_MASK_DECODER;
    if (reads_valid && a->key_valid == nullptr) return fail(TSFM_E_INVALID, "mask %d needs key_valid", a->mask);
    if (a->kv_batch < 0) return fail(TSFM_E_INVALID, "negative kv_batch");
    if (a->q_pos0 < 0) return fail(TSFM_E_INVALID, "negative q_pos0");
    if (a->mask == TSFM_MASK_DECODER && (a->ctx_keys < 0 || a->chain_start < 0))
        return fail(TSFM_E_INVALID, "negative decoder bounds");
    if (a->bias != nullptr && a->rel_table != nullptr) return fail(TSFM_E_INVALID, "both dense and T5 bias given");
    if (a->bias != nullptr && (a->bias_head < 0 || a->bias_row < 0)) return fail(TSFM_E_INVALID, "negative bias stride");
    if (a->bias != nullptr && span_checked(a->heads, a->n_q, a->bias_row, a->bias_head, a->n_k) < 0)
        return fail(TSFM_E_UNSUPPORTED, "the bias view spans more than 2^46 elements");
    if (a->kv_batch > kMaxSpan) return fail(TSFM_E_UNSUPPORTED, "kv_batch past 2^46");
    if (a->rel_table != nullptr) {
        if (a->rel_bucket == nullptr || a->rel_buckets <= 0) return fail(TSFM_E_INVALID, "T5 bias needs rel_bucket");
        if (a->q_pos0 != 0) return fail(TSFM_E_UNSUPPORTED, "T5 bias needs q_pos0 == 0");
        if ((int64_t)a->n_q + a->n_k - 1 > tsfm::kRelMax)
            return fail(TSFM_E_UNSUPPORTED, "T5 bias supports n_q + n_k - 1 <= %d", tsfm::kRelMax);
    }
    if (a->rope_cos != nullptr) {
        if (a->rope_sin == nullptr) return fail(TSFM_E_INVALID, "rope_sin is NULL");
        if (a->rope_half != a->head_dim / 2) return fail(TSFM_E_UNSUPPORTED, "rope_half must be head_dim / 2");
        if (a->rope_rows_per_table < 0 || a->rope_row0 < 0 || a->rope_table_stride < 0)
            return fail(TSFM_E_INVALID, "bad rope table layout");
        if (a->rope_table_stride % 4) return fail(TSFM_E_UNSUPPORTED, "rope_table_stride must be a multiple of 4");
    }
    if (a->flags & TSFM_ATTN_DEVICE_PTRS) {
        if (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16) || !aligned(a->o, 16))
            return fail(TSFM_E_UNSUPPORTED, "device q/k/v/o must be 16-byte aligned");
        if (a->rope_cos != nullptr && (!aligned(a->rope_cos, 16) || !aligned(a->rope_sin, 16)))
            return fail(TSFM_E_UNSUPPORTED, "device RoPE tables must be 16-byte aligned");
    }
    return TSFM_OK;
}

int launch(const tsfm_attn_args* a, const tsfm::Params& p, hipStream_t s) {
    const int bias = a->rel_table != nullptr ? tsfm::BIAS_REL : (a->bias != nullptr ? tsfm::BIAS_DENSE : tsfm::BIAS_NONE);
    const bool rope = a->rope_cos != nullptr;
    hipError_t e;
    if (a->dtype == TSFM_DTYPE_F32) e = tsfm::launch_attn_f32(p, a->mask, bias, rope, s);
    else e = tsfm::launch_attn_half(p, a->dtype == TSFM_DTYPE_BF16, a->mask, bias, rope, s);
    if (e != hipSuccess) return hip_fail(e, "attention kernel launch");
    return TSFM_OK;
}

tsfm::Params params_from(const tsfm_attn_args* a) {
    tsfm::Params p{};
    p.q = a->q; p.k = a->k; p.v = a->v; p.o = a->o;
    p.q_tok = a->q_tok; p.q_batch = a->q_batch; p.k_tok = a->k_tok; p.k_batch = a->k_batch;
    p.v_tok = a->v_tok; p.v_batch = a->v_batch; p.o_tok = a->o_tok; p.o_batch = a->o_batch;
    p.key_valid = a->key_valid; p.kv_batch = a->kv_batch;
    p.bias = a->bias; p.bias_head = a->bias_head; p.bias_row = a->bias_row;
    p.rel_table = a->rel_table; p.rel_bucket = a->rel_bucket; p.rel_buckets = a->rel_buckets;
    p.rope_cos = a->rope_cos; p.rope_sin = a->rope_sin;
    p.rope_table_stride = a->rope_table_stride; p.rope_rows_per_table = a->rope_rows_per_table;
    p.rope_row0 = a->rope_row0;
    p.B = a->batch; p.H = a->heads; p.n_q = a->n_q; p.n_k = a->n_k; p.q_pos0 = a->q_pos0;
    p.ctx_keys = a->ctx_keys; p.chain_start = a->chain_start; p.scale = a->scale;
    return p;
}

}  // namespace

extern "C" {

int tsfm_attn_init(void) { return ensure_ready(); }

int tsfm_attn_available(void) { return ensure_ready() == TSFM_OK ? 1 : 0; }

const char* tsfm_attn_last_error(void) { return t_err; }

uint32_t tsfm_t5_relative_bucket(int64_t rel, uint32_t num_buckets, uint32_t max_distance) {
    // T5 bidirectional bucket with a float32 log (src/chronos_bolt/model.zig:74-85).
    const uint32_t half = num_buckets / 2;
    const uint32_t base = rel > 0 ? half : 0;
    const uint32_t rp = (uint32_t)(rel < 0 ? -rel : rel);
    const uint32_t max_exact = half / 2;
    if (rp < max_exact) return base + rp;
    const float ratio = (float)rp / (float)max_exact;
    const float denom = (float)std::log((double)max_distance / (double)max_exact);
    const float large_f = std::log(ratio) / denom * (float)(half - max_exact);
    const uint32_t large = max_exact + (uint32_t)large_f;
    return base + (large < half - 1 ? large : half - 1);
}

int tsfm_t5_bucket_table(int32_t* out, int32_t n_q, int32_t n_k, uint32_t num_buckets, uint32_t max_distance) {
    if (out == nullptr || n_q <= 0 || n_k <= 0 || num_buckets < 4)
        return fail(TSFM_E_INVALID, "bad bucket table request");
    const int64_t n = (int64_t)n_q + n_k - 1;
    for (int64_t t = 0; t < n; t++)
        out[t] = (int32_t)tsfm_t5_relative_bucket(t - (n_q - 1), num_buckets, max_distance);
    return TSFM_OK;
}

int tsfm_attn_fwd(const tsfm_attn_args* a) {
    int rc = validate(a);
    if (rc != TSFM_OK) return rc;
    if (a->batch == 0 || a->heads == 0 || a->n_q == 0) return TSFM_OK;  // nothing to compute
    if (a->n_k == 0) return fail(TSFM_E_INVALID, "n_k is 0 with queries present");
    rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");

    tsfm::Params p = params_from(a);
    if (a->flags & TSFM_ATTN_DEVICE_PTRS) return launch(a, p, static_cast<hipStream_t>(a->stream));

    // Host pointers: stage every input, run, copy the output rows back, synchronise.
    const int64_t B = a->batch, H = a->heads, D = a->head_dim, row = H * D;
    const size_t es = elem_size(a->dtype);
    const bool reads_valid = a->mask == TSFM_MASK_KEYS_ADDITIVE || a->mask == TSFM_MASK_CAUSAL_KEYS ||
                             a->mask == TSFM_MASK_FULL_KEYS || a->mask == TSFM_MASK_DECODER;
    const size_t q_n = span(B, a->n_q, a->q_tok, a->q_batch, row) * es;
    const size_t k_n = span(B, a->n_k, a->k_tok, a->k_batch, row) * es;
    const size_t v_n = span(B, a->n_k, a->v_tok, a->v_batch, row) * es;
    const size_t o_n = span(B, a->n_q, a->o_tok, a->o_batch, row) * es;
    const int64_t kv_len = a->mask == TSFM_MASK_DECODER ? (a->ctx_keys < a->n_k ? a->ctx_keys : a->n_k) : a->n_k;
    const size_t kv_n = reads_valid && kv_len > 0 ? (size_t)span(B, 1, 0, a->kv_batch, kv_len) : 0;
    const size_t bias_n = a->bias ? (size_t)((H - 1) * a->bias_head + (a->n_q - 1) * a->bias_row + a->n_k) * 4 : 0;
    const size_t relt_n = a->rel_table ? (size_t)a->rel_buckets * H * 4 : 0;
    const size_t relb_n = a->rel_table ? (size_t)(a->n_q + a->n_k - 1) * 4 : 0;
    int64_t ntab = 1;
    if (a->rope_cos != nullptr && a->rope_rows_per_table > 0)
        ntab = (a->rope_row0 + B - 1) / a->rope_rows_per_table + 1;
    const int64_t npos = a->n_k > a->q_pos0 + a->n_q ? a->n_k : a->q_pos0 + a->n_q;
    const size_t rope_n = a->rope_cos ? (size_t)((ntab - 1) * a->rope_table_stride + npos * a->rope_half) * 4 : 0;

    Plan plan;
    const size_t q_at = plan.take(q_n), k_at = plan.take(k_n), v_at = plan.take(v_n), o_at = plan.take(o_n);
    const size_t kv_at = plan.take(kv_n), bias_at = plan.take(bias_n), relt_at = plan.take(relt_n);
    const size_t relb_at = plan.take(relb_n), rc_at = plan.take(rope_n), rs_at = plan.take(rope_n);
    rc = ensure_buf(ctx, plan.off);
    if (rc != TSFM_OK) return rc;

    // Bucket ids index the bias table on the device: check them here, where they are readable.
    if (a->rel_table != nullptr)
        for (int64_t t = 0; t < a->n_q + a->n_k - 1; t++)
            if (a->rel_bucket[t] < 0 || a->rel_bucket[t] >= a->rel_buckets)
                return fail(TSFM_E_INVALID, "rel_bucket[%lld] = %d outside [0, %d)", (long long)t, a->rel_bucket[t],
                            a->rel_buckets);

    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    struct Up { const void* src; size_t at, n; } ups[] = {
        {a->q, q_at, q_n}, {a->k, k_at, k_n}, {a->v, v_at, v_n}, {a->key_valid, kv_at, kv_n},
        {a->bias, bias_at, bias_n}, {a->rel_table, relt_at, relt_n}, {a->rel_bucket, relb_at, relb_n},
        {a->rope_cos, rc_at, rope_n}, {a->rope_sin, rs_at, rope_n}};
    for (const Up& u : ups) {
        if (u.n == 0 || u.src == nullptr) continue;
        hipError_t e = hipMemcpyAsync(base + u.at, u.src, u.n, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return hip_fail(e, "host-to-device copy");
    }
    p.q = base + q_at; p.k = base + k_at; p.v = base + v_at; p.o = base + o_at;
    p.key_valid = kv_n > 0 ? reinterpret_cast<const uint8_t*>(base + kv_at) : nullptr;
    if (a->bias) p.bias = reinterpret_cast<const float*>(base + bias_at);
    if (a->rel_table) {
        p.rel_table = reinterpret_cast<const float*>(base + relt_at);
        p.rel_bucket = reinterpret_cast<const int32_t*>(base + relb_at);
    }
    if (a->rope_cos) {
        p.rope_cos = reinterpret_cast<const float*>(base + rc_at);
        p.rope_sin = reinterpret_cast<const float*>(base + rs_at);
    }
    rc = launch(a, p, s);
    if (rc != TSFM_OK) {
        (void)hipStreamSynchronize(s);
        return rc;
    }
    hipError_t e = copy_rows_d2h(a->o, base + o_at, B, a->n_q, a->o_batch * es, a->o_tok * es, row * es, s);
    if (e != hipSuccess) return hip_fail(e, "device-to-host copy");
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

// ---- Timestral variate attention ----------------------------------------------------------------

static_assert(tsfm::kVariateMaxRows == TSFM_VARIATE_MAX_ROWS, "the kernels' role words cover the ABI's rows");

int tsfm_variate_attend(const tsfm_variate_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (a->dtype != TSFM_DTYPE_F32) return fail(TSFM_E_UNSUPPORTED, "variate attention is f32 only");
    if (a->head_dim != 64) return fail(TSFM_E_UNSUPPORTED, "head_dim %d (supported: 64)", a->head_dim);
    if (a->groups < 0 || a->vall < 0 || a->n_tok < 0 || a->n_enc < 0 || a->heads < 0)
        return fail(TSFM_E_INVALID, "negative size");
    if (a->vall > TSFM_VARIATE_MAX_ROWS)
        return fail(TSFM_E_UNSUPPORTED, "vall %d (supported: up to %d rows per series)", a->vall, TSFM_VARIATE_MAX_ROWS);
    if (a->n_enc > a->n_tok) return fail(TSFM_E_INVALID, "n_enc %d > n_tok %d", a->n_enc, a->n_tok);
    if (a->qkv == nullptr || a->o == nullptr) return fail(TSFM_E_INVALID, "qkv and o are required");
    if (a->cov != 0 && a->roles == nullptr && a->vall > 0) return fail(TSFM_E_INVALID, "roles is required with cov");
    if (a->roles != nullptr)
        for (int32_t i = 0; i < a->vall; i++)
            if (a->roles[i] > TSFM_ROLE_KNOWN) return fail(TSFM_E_INVALID, "roles[%d] = %d", i, a->roles[i]);
    if (a->n_enc > 0 && a->vall > 1 && a->key_valid == nullptr) return fail(TSFM_E_INVALID, "key_valid is required");
    if (a->qkv_row < 0 || a->qkv_tok < 0 || a->o_row < 0 || a->o_tok < 0 || a->gate_row < 0 || a->gate_tok < 0 ||
        a->kv_row < 0)
        return fail(TSFM_E_INVALID, "negative stride");
    if (a->key_valid != nullptr && a->kv_row < a->n_enc && a->groups * a->vall > 1)
        return fail(TSFM_E_INVALID, "kv_row %lld shorter than n_enc %d", (long long)a->kv_row, a->n_enc);
    if (a->qkv_row % 4 || a->qkv_tok % 4 || a->o_row % 4 || a->o_tok % 4 || a->gate_row % 4 || a->gate_tok % 4)
        return fail(TSFM_E_UNSUPPORTED, "strides must be multiples of 16 bytes");
    {
        const int64_t rows = (int64_t)a->groups * a->vall, D = (int64_t)a->heads * a->head_dim;
        if (span_checked(rows, a->n_tok, a->qkv_tok, a->qkv_row, 3 * D) < 0 ||
            span_checked(rows, a->n_tok, a->o_tok, a->o_row, D) < 0 ||
            (a->gate != nullptr && span_checked(rows, a->n_tok, a->gate_tok, a->gate_row, D) < 0) ||
            (a->key_valid != nullptr && span_checked(rows, 1, 0, a->kv_row, a->n_enc) < 0))
            return fail(TSFM_E_UNSUPPORTED, "a view spans more than 2^46 elements");
    }
    if (a->groups == 0 || a->vall == 0 || a->n_tok == 0 || a->heads == 0) return TSFM_OK;  // nothing to compute
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");

    tsfm::VariateParams p{};
    p.qkv = static_cast<const float*>(a->qkv); p.qkv_row = a->qkv_row; p.qkv_tok = a->qkv_tok;
    p.o = static_cast<float*>(a->o); p.o_row = a->o_row; p.o_tok = a->o_tok;
    p.gate = static_cast<const float*>(a->gate); p.gate_row = a->gate_row; p.gate_tok = a->gate_tok;
    p.key_valid = a->key_valid; p.kv_row = a->kv_row;
    if (a->roles != nullptr)
        for (int i = 0; i < a->vall; i++) p.roles[i >> 2] |= (uint32_t)a->roles[i] << (8 * (i & 3));
    p.groups = a->groups; p.vall = a->vall; p.n_tok = a->n_tok; p.n_enc = a->n_enc; p.heads = a->heads;
    p.cov = a->cov != 0; p.scale = a->scale;
    hipError_t e;
    if (a->flags & TSFM_ATTN_DEVICE_PTRS) {
        if (!aligned(a->qkv, 16) || !aligned(a->o, 16) || (a->gate != nullptr && !aligned(a->gate, 16)))
            return fail(TSFM_E_UNSUPPORTED, "device qkv/o/gate must be 16-byte aligned");
        e = tsfm::launch_variate(p, static_cast<hipStream_t>(a->stream));
        if (e != hipSuccess) return hip_fail(e, "variate attention launch");
        return TSFM_OK;
    }
    // Host pointers: stage every input, run, copy the output rows back, synchronise.
    const int64_t rows = (int64_t)a->groups * a->vall, D = (int64_t)a->heads * a->head_dim;
    const size_t qkv_n = span(rows, a->n_tok, a->qkv_tok, a->qkv_row, 3 * D) * 4;
    const size_t o_n = span(rows, a->n_tok, a->o_tok, a->o_row, D) * 4;
    const size_t g_n = a->gate ? span(rows, a->n_tok, a->gate_tok, a->gate_row, D) * 4 : 0;
    const size_t kv_n = a->key_valid && a->n_enc > 0 ? (size_t)span(rows, 1, 0, a->kv_row, a->n_enc) : 0;
    Plan plan;
    const size_t qkv_at = plan.take(qkv_n), o_at = plan.take(o_n), g_at = plan.take(g_n), kv_at = plan.take(kv_n);
    rc = ensure_buf(ctx, plan.off);
    if (rc != TSFM_OK) return rc;
    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    struct Up { const void* src; size_t at, n; } ups[] = {
        {a->qkv, qkv_at, qkv_n}, {a->gate, g_at, g_n}, {a->key_valid, kv_at, kv_n}};
    for (const Up& u : ups) {
        if (u.n == 0 || u.src == nullptr) continue;
        if ((e = hipMemcpyAsync(base + u.at, u.src, u.n, hipMemcpyHostToDevice, s)) != hipSuccess)
            return hip_fail(e, "host-to-device copy");
    }
    p.qkv = reinterpret_cast<const float*>(base + qkv_at);
    p.o = reinterpret_cast<float*>(base + o_at);
    if (a->gate) p.gate = reinterpret_cast<const float*>(base + g_at);
    p.key_valid = kv_n > 0 ? reinterpret_cast<const uint8_t*>(base + kv_at) : nullptr;
    e = tsfm::launch_variate(p, s);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "variate attention launch");
    }
    if ((e = copy_rows_d2h(a->o, base + o_at, rows, a->n_tok, a->o_row * 4, a->o_tok * 4, D * 4, s)) != hipSuccess)
        return hip_fail(e, "device-to-host copy");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

// ---- fused projection ---------------------------------------------------------------------------

}  // extern "C"

namespace {

// Validates a projection request and fills the kernel parameters with the caller's pointers.
// Returns TSFM_OK, a non-zero error code, or kNothing when the product is empty.
constexpr int kNothing = -1;
int proj_request(const tsfm_proj_args* a, tsfm::ProjParams* pp) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (a->dtype != TSFM_DTYPE_F32) return fail(TSFM_E_UNSUPPORTED, "the projection computes in f32 only");
    if (a->out_dtype < TSFM_DTYPE_F32 || a->out_dtype > TSFM_DTYPE_F16)
        return fail(TSFM_E_INVALID, "bad out_dtype %d", a->out_dtype);
    if (a->head_dim != 64) return fail(TSFM_E_UNSUPPORTED, "head_dim %d (supported: 64)", a->head_dim);
    if (a->batch < 0 || a->seq < 0 || a->d_in < 0 || a->heads < 0) return fail(TSFM_E_INVALID, "negative size");
    if (a->x == nullptr || a->w_q == nullptr || a->w_k == nullptr || a->w_v == nullptr || a->q == nullptr ||
        a->k == nullptr || a->v == nullptr)
        return fail(TSFM_E_INVALID, "x, w_q, w_k, w_v, q, k and v are required");
    if ((a->w_gate == nullptr) != (a->gate == nullptr)) return fail(TSFM_E_INVALID, "w_gate and gate go together");
    if ((a->rope_cos == nullptr) != (a->rope_sin == nullptr))
        return fail(TSFM_E_INVALID, "rope_cos and rope_sin go together");
    const int64_t width = (int64_t)a->heads * a->head_dim;
    const bool gated = a->gate != nullptr, rope = a->rope_cos != nullptr;
    if (a->x_tok < a->d_in || a->q_tok < width || a->k_tok < width || a->v_tok < width ||
        (gated && a->gate_tok < width))
        return fail(TSFM_E_INVALID, "a token stride is shorter than its row");
    if (rope && (a->rope_half != a->head_dim / 2 || a->rope_rows_per_table < 0 || a->rope_row0 < 0 ||
                 a->rope_table_stride < 0))
        return fail(TSFM_E_INVALID, "bad RoPE table description");
    const int64_t tokens = (int64_t)a->batch * a->seq;
    if (tokens == 0 || width == 0) return kNothing;
    if (a->d_in == 0 || a->d_in % 16) return fail(TSFM_E_UNSUPPORTED, "d_in %d (supported: multiples of 16)", a->d_in);
    if (tokens > 0x7fffffff || 4 * width > 0x7fffffff) return fail(TSFM_E_UNSUPPORTED, "too many tokens or heads");
    if (span_checked(1, tokens, a->x_tok, 0, a->d_in) < 0 || span_checked(1, tokens, a->q_tok, 0, width) < 0 ||
        span_checked(1, tokens, a->k_tok, 0, width) < 0 || span_checked(1, tokens, a->v_tok, 0, width) < 0 ||
        (gated && span_checked(1, tokens, a->gate_tok, 0, width) < 0) ||
        (rope && span_checked(1, (int64_t)a->rope_row0 + a->batch, a->rope_table_stride, 0,
                              (int64_t)a->seq * a->rope_half) < 0))
        return fail(TSFM_E_UNSUPPORTED, "a view spans more than 2^46 elements");
    if (a->x_tok % 4 || a->q_tok % 4 || a->k_tok % 4 || a->v_tok % 4 || (gated && a->gate_tok % 4) ||
        (rope && a->rope_table_stride % 4))
        return fail(TSFM_E_UNSUPPORTED, "strides must be multiples of 16 bytes");
    tsfm::ProjParams p{};
    p.x = a->x; p.x_tok = a->x_tok;
    p.w0 = a->w_q; p.w1 = a->w_k; p.w2 = a->w_v; p.w3 = a->w_gate;
    p.w_ld = a->d_in; p.alpha = 1.f; p.epi = tsfm::kEpiNone;
    p.y0 = a->q; p.y1 = a->k; p.y2 = a->v; p.y3 = a->gate;
    p.out_dtype = a->out_dtype;
    p.y0_tok = a->q_tok; p.y1_tok = a->k_tok; p.y2_tok = a->v_tok; p.y3_tok = a->gate_tok;
    p.rope_cos = a->rope_cos; p.rope_sin = a->rope_sin;
    p.rope_table_stride = a->rope_table_stride;
    p.rope_rows_per_table = a->rope_rows_per_table; p.rope_row0 = a->rope_row0;
    p.tokens = (int32_t)tokens; p.seq = a->seq; p.d_in = a->d_in; p.width = (int32_t)width;
    p.n_out = gated ? 4 : 3;
    *pp = p;
    return TSFM_OK;
}

bool device_ptrs_aligned(const tsfm_proj_args* a) {
    const void* ptrs[] = {a->x, a->w_q, a->w_k, a->w_v, a->w_gate, a->q, a->k, a->v, a->gate, a->rope_cos,
                          a->rope_sin};
    for (const void* q : ptrs)
        if (q != nullptr && !aligned(q, 16)) return false;
    return true;
}

// The split partials of tsfm_qkv_project_noalloc: one copy per GPU in the code object's device
// memory, so the call allocates nothing. Its address on each device is looked up once, with that
// device current (the array's name is only a host-side stand-in for it).
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_at[kMaxDevices] = {};

hipError_t noalloc_scratch(void** out) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_at[device] == nullptr) {
        void* ptr = nullptr;
        if ((e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) != hipSuccess) return e;
        if (ptr == nullptr) return hipErrorInvalidSymbol;
        g_scratch_at[device] = ptr;
    }
    *out = g_scratch_at[device];
    return hipSuccess;
}

}  // namespace

extern "C" {

int tsfm_qkv_project_noalloc(const tsfm_proj_args* a) {
    tsfm::ProjParams p{};
    int rc = proj_request(a, &p);
    if (rc == kNothing) return TSFM_OK;
    if (rc != TSFM_OK) return rc;
    if (!(a->flags & TSFM_ATTN_DEVICE_PTRS))
        return fail(TSFM_E_UNSUPPORTED, "tsfm_qkv_project_noalloc takes device pointers only");
    if (!device_ptrs_aligned(a)) return fail(TSFM_E_UNSUPPORTED, "device pointers must be 16-byte aligned");
    tsfm::ProjParams plan = p;
    const size_t need = tsfm::proj_split_bytes(plan);
    if (need > kNoAllocScratchBytes)
        return fail(TSFM_E_UNSUPPORTED,
                    "this product's split partials need %zu bytes; tsfm_qkv_project_noalloc holds %zu "
                    "(use tsfm_qkv_project)", need, kNoAllocScratchBytes);
    if ((rc = ensure_ready()) != TSFM_OK) return rc;
    void* part = nullptr;
    hipError_t e = noalloc_scratch(&part);
    if (e != hipSuccess) return hip_fail(e, "scratch symbol address");
    tsfm::SplitWorkspace ws(static_cast<float*>(part));
    e = tsfm::launch_proj(p, static_cast<hipStream_t>(a->stream));
    if (e != hipSuccess) return hip_fail(e, "projection launch");
    return TSFM_OK;
}

int tsfm_qkv_project(const tsfm_proj_args* a) {
    tsfm::ProjParams p{};
    int rc = proj_request(a, &p);
    if (rc == kNothing) return TSFM_OK;
    if (rc != TSFM_OK) return rc;
    const int64_t width = (int64_t)a->heads * a->head_dim, tokens = (int64_t)a->batch * a->seq;
    const bool gated = a->gate != nullptr, rope = a->rope_cos != nullptr;
    if ((rc = ensure_ready()) != TSFM_OK) return rc;
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    const int64_t oes = (int64_t)elem_size(a->out_dtype);
    hipError_t e;
    if (a->flags & TSFM_ATTN_DEVICE_PTRS) {
        if (!device_ptrs_aligned(a)) return fail(TSFM_E_UNSUPPORTED, "device pointers must be 16-byte aligned");
        hipStream_t s = static_cast<hipStream_t>(a->stream);
        float* part = nullptr;
        bool owned = false;
        if ((e = split_buf_for(ctx, s, &part, &owned)) != hipSuccess) return hip_fail(e, "split workspace");
        const size_t planes_n = tsfm::proj_plane_bytes(tokens, a->d_in, width * (gated ? 4 : 3));
        char* planes = nullptr;
        bool planes_owned = false;
        if ((e = tsfm::abi::scratch_acquire(s, tsfm::abi::kSlotProject, planes_n, &planes, &planes_owned)) != hipSuccess) {
            if (owned) (void)hipFreeAsync(part, s);
            return hip_fail(e, "operand split workspace");
        }
        {
            tsfm::SplitWorkspace ws(part);
            tsfm::PlaneWorkspace pws(planes, planes_n);
            e = tsfm::launch_proj(p, s);
        }
        const hipError_t f = owned ? hipFreeAsync(part, s) : hipSuccess;
        const hipError_t g = planes_owned ? hipFreeAsync(planes, s) : hipSuccess;
        if (e != hipSuccess) return hip_fail(e, "projection launch");
        if (f != hipSuccess) return hip_fail(f, "split workspace release");
        if (g != hipSuccess) return hip_fail(g, "operand split workspace release");
        return TSFM_OK;
    }
    // Host pointers: stage x, the weights and the tables, run, copy the output rows back.
    const size_t x_n = (size_t)span(1, tokens, a->x_tok, 0, a->d_in) * 4;
    const size_t w_n = (size_t)(width * a->d_in) * 4;
    const size_t y_n[4] = {(size_t)(span(1, tokens, a->q_tok, 0, width) * oes),
                           (size_t)(span(1, tokens, a->k_tok, 0, width) * oes),
                           (size_t)(span(1, tokens, a->v_tok, 0, width) * oes),
                           gated ? (size_t)(span(1, tokens, a->gate_tok, 0, width) * oes) : 0};
    size_t t_n = 0;
    if (rope) {
        const int64_t last = a->rope_rows_per_table > 0 ? (a->rope_row0 + a->batch - 1) / a->rope_rows_per_table : 0;
        t_n = (size_t)(last * a->rope_table_stride + (int64_t)a->seq * a->rope_half) * 4;
    }
    Plan plan;
    const size_t x_at = plan.take(x_n);
    size_t w_at[4], y_at[4];
    for (int i = 0; i < 4; i++) w_at[i] = plan.take(i < 3 || gated ? w_n : 0);
    for (int i = 0; i < 4; i++) y_at[i] = plan.take(y_n[i]);
    const size_t c_at = plan.take(t_n), s_at = plan.take(t_n), part_at = plan.take(tsfm::kSplitWorkspaceBytes);
    const size_t planes_n = tsfm::proj_plane_bytes(tokens, a->d_in, width * (gated ? 4 : 3));
    const size_t planes_at = plan.take(planes_n);
    rc = ensure_buf(ctx, plan.off);
    if (rc != TSFM_OK) return rc;
    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    tsfm::SplitWorkspace ws(reinterpret_cast<float*>(base + part_at));
    tsfm::PlaneWorkspace pws(base + planes_at, planes_n);
    const float* w_src[4] = {a->w_q, a->w_k, a->w_v, a->w_gate};
    struct Up { const void* src; size_t at, n; } ups[] = {
        {a->x, x_at, x_n}, {w_src[0], w_at[0], w_n}, {w_src[1], w_at[1], w_n}, {w_src[2], w_at[2], w_n},
        {w_src[3], w_at[3], gated ? w_n : 0}, {a->rope_cos, c_at, t_n}, {a->rope_sin, s_at, t_n}};
    for (const Up& u : ups) {
        if (u.n == 0 || u.src == nullptr) continue;
        if ((e = hipMemcpyAsync(base + u.at, u.src, u.n, hipMemcpyHostToDevice, s)) != hipSuccess)
            return hip_fail(e, "host-to-device copy");
    }
    p.x = reinterpret_cast<const float*>(base + x_at);
    p.w0 = reinterpret_cast<const float*>(base + w_at[0]);
    p.w1 = reinterpret_cast<const float*>(base + w_at[1]);
    p.w2 = reinterpret_cast<const float*>(base + w_at[2]);
    p.w3 = gated ? reinterpret_cast<const float*>(base + w_at[3]) : nullptr;
    p.y0 = base + y_at[0];
    p.y1 = base + y_at[1];
    p.y2 = base + y_at[2];
    p.y3 = gated ? base + y_at[3] : nullptr;
    if (rope) {
        p.rope_cos = reinterpret_cast<const float*>(base + c_at);
        p.rope_sin = reinterpret_cast<const float*>(base + s_at);
    }
    e = tsfm::launch_proj(p, s);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "projection launch");
    }
    void* const dst[4] = {a->q, a->k, a->v, a->gate};
    const int64_t tok[4] = {a->q_tok, a->k_tok, a->v_tok, a->gate_tok};
    for (int i = 0; i < (gated ? 4 : 3); i++)
        if ((e = copy_rows_d2h(dst[i], base + y_at[i], 1, tokens, 0, tok[i] * oes, width * oes, s)) != hipSuccess)
            return hip_fail(e, "device-to-host copy");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

// ---- Chronos-2 encoder stack ----------------------------------------------------------------------

namespace {

// One nn.linear on the matrix cores: y = x w^T over rows tokens, with an optional ReLU or residual
// (y = resid + x w^T) epilogue.
hipError_t linear_on(const float* x, int64_t x_tok, const float* w, int out, int in, float* y, int64_t y_tok,
                     int rows, int epi, const float* resid, hipStream_t s, const float* bias = nullptr,
                     const void* x_pre = nullptr, void* y_planes = nullptr) {
    tsfm::ProjParams p{};
    p.x = x; p.x_tok = x_tok; p.w0 = w; p.w_ld = in; p.alpha = 1.f; p.epi = epi; p.bias = bias;
    p.resid = resid; p.resid_tok = y_tok;
    p.y0 = y; p.y0_tok = y_tok;
    p.tokens = rows; p.seq = rows; p.d_in = in; p.width = out; p.n_out = 1; p.out_dtype = TSFM_DTYPE_F32;
    p.x_pre = x_pre; p.y_planes = y_planes;
    return tsfm::launch_proj(p, s);
}

// linear_on with the input rows normalised as they are loaded (x read as rmsNorm(x, in_scale, eps)):
// products of at most 16 rows (tsfm::proj_fuses_input_norm), one launch fewer than the norm first.
hipError_t linear_in_norm_on(const float* x, int64_t x_tok, const float* in_scale, float eps, const float* w, int out,
                             int in, float* y, int64_t y_tok, int rows, int epi, hipStream_t s) {
    tsfm::ProjParams p{};
    p.x = x; p.x_tok = x_tok; p.w0 = w; p.w_ld = in; p.alpha = 1.f; p.epi = epi;
    p.y0 = y; p.y0_tok = y_tok;
    p.tokens = rows; p.seq = rows; p.d_in = in; p.width = out; p.n_out = 1; p.out_dtype = TSFM_DTYPE_F32;
    p.in_norm_scale = in_scale; p.in_norm_eps = eps;
    return tsfm::launch_proj(p, s);
}

// TSFM_UNFUSED_NORM=1 makes linear_norm_on queue the product and the row norm as two launches: the
// form the fused one must equal bit for bit (a diagnostic switch; same arithmetic either way).
bool unfused_norm_requested() {
    const char* e = getenv("TSFM_UNFUSED_NORM");
    return e != nullptr && e[0] != '\0' && strcmp(e, "0") != 0;
}

// linear_on followed by nn.rmsNorm of the finished rows into norm_out (may be y): one launch fewer
// when the product splits its reduction (the reduce normalises the rows), the same bits either way.
hipError_t linear_norm_on(const float* x, int64_t x_tok, const float* w, int out, int in, float* y, int64_t y_tok,
                          int rows, int epi, const float* resid, const float* norm_scale, float* norm_out,
                          int64_t norm_tok, float eps, hipStream_t s) {
    if (unfused_norm_requested()) {
        const hipError_t e = linear_on(x, x_tok, w, out, in, y, y_tok, rows, epi, resid, s);
        if (e != hipSuccess) return e;
        return tsfm::launch_rms_norm(y, y_tok, norm_out, norm_tok, norm_scale, rows, out, eps, s);
    }
    tsfm::ProjParams p{};
    p.x = x; p.x_tok = x_tok; p.w0 = w; p.w_ld = in; p.alpha = 1.f; p.epi = epi;
    p.resid = resid; p.resid_tok = y_tok;
    p.y0 = y; p.y0_tok = y_tok;
    p.tokens = rows; p.seq = rows; p.d_in = in; p.width = out; p.n_out = 1; p.out_dtype = TSFM_DTYPE_F32;
    p.norm_scale = norm_scale; p.norm_out = norm_out; p.norm_out_tok = norm_tok; p.norm_eps = eps;
    return tsfm::launch_proj(p, s);
}

// The layer loop on device buffers. scratch: xn, q, k, v, ab (rows x d each), then h (rows x d_ff).
// encode_on's scratch: x_norm, q, k, v, the attention output and the MLP hidden rows in f32, then
// the pre-split x_norm, group values and MLP hidden rows of the fused path.
size_t encode_scratch_bytes(int64_t rows, int64_t d, int64_t F) {
    return (size_t)(rows * (5 * d + F)) * 4 + 2 * tsfm::plane_operand_bytes(rows, d) +
           tsfm::plane_operand_bytes(rows, F);
}

hipError_t encode_on(const tsfm_chronos2_encode_args* a, float* x, const uint8_t* kv, const float* cs,
                     const float* sn, const tsfm_chronos2_layer* layers, const float* final_norm, float* scratch,
                     hipStream_t s) {
    const int64_t d = a->d_model, rows = (int64_t)a->batch * a->seq;
    float* xn = scratch;
    float* q = xn + rows * d;
    float* k = q + rows * d;
    float* v = k + rows * d;
    float* ab = v + rows * d;
    float* h = ab + rows * d;
    const int R = (int)rows, D = (int)d, F = a->d_ff;
    // With a PlaneWorkspace for these products, the row norms and the group-value and MLP-input
    // products write their results split into bf16 parts (after the f32 scratch,
    // encode_scratch_bytes), and the products after them read those parts directly: no f32 round
    // trip and no separate split for x.
    const bool fused = d % 32 == 0 && F % 32 == 0 && tsfm::proj_planes_ready(rows, d, d) &&
                       tsfm::proj_planes_ready(rows, d, F) && tsfm::proj_planes_ready(rows, F, d);
    char* const pl = reinterpret_cast<char*>(h + rows * F);
    void* const xn_pl = pl;
    void* const v_pl = pl + tsfm::plane_operand_bytes(rows, d);
    void* const h_pl = pl + 2 * tsfm::plane_operand_bytes(rows, d);
    auto norm = [&](const float* scale) {
        return fused ? tsfm::launch_rms_norm_planes(x, d, xn_pl, scale, R, D, a->eps, s)
                     : tsfm::launch_rms_norm(x, d, xn, d, scale, R, D, a->eps, s);
    };
    hipError_t e = hipSuccess;
    for (int l = 0; l < a->n_layers && e == hipSuccess; l++) {
        const tsfm_chronos2_layer& ly = layers[l];
        // time attention
        if ((e = norm(ly.time_norm)) != hipSuccess) break;
        tsfm::ProjParams p{};
        p.x = xn; p.x_tok = d; p.w0 = ly.time_q; p.w1 = ly.time_k; p.w2 = ly.time_v; p.w_ld = d;
        p.alpha = 1.f; p.epi = tsfm::kEpiNone;
        p.y0 = q; p.y1 = k; p.y2 = v; p.y0_tok = p.y1_tok = p.y2_tok = d;
        p.rope_cos = cs; p.rope_sin = sn;
        p.tokens = R; p.seq = a->seq; p.d_in = D; p.width = D; p.n_out = 3; p.out_dtype = TSFM_DTYPE_F32;
        p.x_pre = fused ? xn_pl : nullptr;
        if ((e = tsfm::launch_proj(p, s)) != hipSuccess) break;
        tsfm::Params ap{};
        ap.q = q; ap.k = k; ap.v = v; ap.o = ab;
        ap.q_tok = ap.k_tok = ap.v_tok = ap.o_tok = d;
        ap.q_batch = ap.k_batch = ap.v_batch = ap.o_batch = (int64_t)a->seq * d;
        ap.key_valid = kv; ap.kv_batch = a->seq;
        ap.B = a->batch; ap.H = a->heads; ap.n_q = a->seq; ap.n_k = a->seq; ap.scale = a->scale;
        const int mask = a->keys_all_valid ? TSFM_MASK_FULL : TSFM_MASK_KEYS_ADDITIVE;  // Mask.pick(false, all, true)
        if ((e = tsfm::launch_attn_f32(ap, mask, tsfm::BIAS_NONE, false, s)) != hipSuccess) break;
        if ((e = linear_on(ab, d, ly.time_o, D, D, x, d, R, tsfm::kEpiResidual, x, s)) != hipSuccess) break;
        // group attention with singleton groups
        if ((e = norm(ly.group_norm)) != hipSuccess) break;
        if ((e = linear_on(xn, d, ly.group_v, D, D, v, d, R, tsfm::kEpiNone, nullptr, s, nullptr,
                           fused ? xn_pl : nullptr, fused ? v_pl : nullptr)) != hipSuccess)
            break;
        if ((e = linear_on(v, d, ly.group_o, D, D, x, d, R, tsfm::kEpiResidual, x, s, nullptr,
                           fused ? v_pl : nullptr)) != hipSuccess)
            break;
        // MLP
        if ((e = norm(ly.mlp_norm)) != hipSuccess) break;
        if ((e = linear_on(xn, d, ly.mlp_wi, F, D, h, F, R, tsfm::kEpiRelu, nullptr, s, nullptr,
                           fused ? xn_pl : nullptr, fused ? h_pl : nullptr)) != hipSuccess)
            break;
        if ((e = linear_on(h, F, ly.mlp_wo, D, F, x, d, R, tsfm::kEpiResidual, x, s, nullptr,
                           fused ? h_pl : nullptr)) != hipSuccess)
            break;
    }
    if (e == hipSuccess) e = tsfm::launch_rms_norm(x, d, x, d, final_norm, R, D, a->eps, s);
    return e;
}

}  // namespace

int tsfm_chronos2_encode(const tsfm_chronos2_encode_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (a->batch < 0 || a->seq < 0 || a->n_layers < 0 || a->heads < 0 || a->d_ff < 0)
        return fail(TSFM_E_INVALID, "negative size");
    if (a->head_dim != 64) return fail(TSFM_E_UNSUPPORTED, "head_dim %d (supported: 64)", a->head_dim);
    if (a->d_model != a->heads * a->head_dim) return fail(TSFM_E_INVALID, "d_model != heads * head_dim");
    if ((int64_t)a->batch * a->seq == 0) return TSFM_OK;  // nothing to compute
    if (a->d_model == 0 || a->d_ff <= 0 || a->d_ff % 16)
        return fail(TSFM_E_UNSUPPORTED, "d_ff %d (supported: positive multiples of 16)", a->d_ff);
    if (a->x == nullptr || a->key_valid == nullptr || a->rope_cos == nullptr || a->rope_sin == nullptr ||
        a->final_norm == nullptr || (a->n_layers > 0 && a->layers == nullptr))
        return fail(TSFM_E_INVALID, "x, key_valid, rope tables, final_norm and layers are required");
    for (int l = 0; l < a->n_layers; l++) {
        const tsfm_chronos2_layer& y = a->layers[l];
        const float* w[] = {y.time_norm, y.time_q, y.time_k, y.time_v, y.time_o, y.group_norm,
                            y.group_v, y.group_o, y.mlp_norm, y.mlp_wi, y.mlp_wo};
        for (const float* p : w)
            if (p == nullptr) return fail(TSFM_E_INVALID, "layer %d has a NULL weight", l);
    }
    const int64_t rows = (int64_t)a->batch * a->seq, d = a->d_model, F = a->d_ff;
    if (rows > 0x7fffffff / 4) return fail(TSFM_E_UNSUPPORTED, "too many tokens");
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    const size_t scratch_n = encode_scratch_bytes(rows, d, F);
    const size_t planes_n = tsfm::proj_plane_bytes(rows, std::max(d, F), std::max(3 * d, F));
    hipError_t e;
    if (a->flags & TSFM_ATTN_DEVICE_PTRS) {
        bool ok = aligned(a->x, 16) && aligned(a->rope_cos, 16) && aligned(a->rope_sin, 16) && aligned(a->final_norm, 16);
        for (int l = 0; l < a->n_layers; l++) {
            const tsfm_chronos2_layer& y = a->layers[l];
            const float* w[] = {y.time_norm, y.time_q, y.time_k, y.time_v, y.time_o, y.group_norm,
                                y.group_v, y.group_o, y.mlp_norm, y.mlp_wi, y.mlp_wo};
            for (const float* p : w) ok = ok && aligned(p, 16);
        }
        if (!ok) return fail(TSFM_E_UNSUPPORTED, "device pointers must be 16-byte aligned");
        hipStream_t s = static_cast<hipStream_t>(a->stream);
        char* scratch = nullptr;
        bool owned = false;
        if ((e = tsfm::abi::scratch_acquire(s, tsfm::abi::kSlotEncode, scratch_n + tsfm::kSplitWorkspaceBytes + planes_n,
                                            &scratch, &owned)) != hipSuccess)
            return hip_fail(e, "encoder scratch allocation");
        {
            tsfm::SplitWorkspace ws(reinterpret_cast<float*>(scratch + scratch_n));
            tsfm::PlaneWorkspace pws(scratch + scratch_n + tsfm::kSplitWorkspaceBytes, planes_n);
            e = encode_on(a, a->x, a->key_valid, a->rope_cos, a->rope_sin, a->layers, a->final_norm,
                          reinterpret_cast<float*>(scratch), s);
        }
        const hipError_t f = owned ? hipFreeAsync(scratch, s) : hipSuccess;
        if (e != hipSuccess) return hip_fail(e, "encoder launch");
        if (f != hipSuccess) return hip_fail(f, "encoder scratch release");
        return TSFM_OK;
    }
    // Host pointers: upload x, the mask, the tables and every weight; run; copy x back.
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    const size_t x_n = (size_t)(rows * d) * 4, kv_n = (size_t)rows, t_n = (size_t)a->seq * 32 * 4;
    const size_t dd = (size_t)(d * d) * 4, df = (size_t)(d * F) * 4, vn = (size_t)d * 4;
    const size_t sizes[11] = {vn, dd, dd, dd, dd, vn, dd, dd, vn, df, df};
    Plan plan;
    const size_t x_at = plan.take(x_n), kv_at = plan.take(kv_n), c_at = plan.take(t_n), s_at = plan.take(t_n);
    const size_t fn_at = plan.take(vn), scr_at = plan.take(scratch_n), part_at = plan.take(tsfm::kSplitWorkspaceBytes);
    const size_t planes_at = plan.take(planes_n);
    std::vector<size_t> w_at((size_t)a->n_layers * 11);
    for (int l = 0; l < a->n_layers; l++)
        for (int i = 0; i < 11; i++) w_at[(size_t)l * 11 + i] = plan.take(sizes[i]);
    rc = ensure_buf(ctx, plan.off);
    if (rc != TSFM_OK) return rc;
    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    tsfm::SplitWorkspace ws(reinterpret_cast<float*>(base + part_at));
    tsfm::PlaneWorkspace pws(base + planes_at, planes_n);
    auto up = [&](size_t at, const void* src, size_t n) {
        return hipMemcpyAsync(base + at, src, n, hipMemcpyHostToDevice, s);
    };
    if ((e = up(x_at, a->x, x_n)) != hipSuccess || (e = up(kv_at, a->key_valid, kv_n)) != hipSuccess ||
        (e = up(c_at, a->rope_cos, t_n)) != hipSuccess || (e = up(s_at, a->rope_sin, t_n)) != hipSuccess ||
        (e = up(fn_at, a->final_norm, vn)) != hipSuccess)
        return hip_fail(e, "host-to-device copy");
    std::vector<tsfm_chronos2_layer> dev_layers((size_t)a->n_layers);
    for (int l = 0; l < a->n_layers; l++) {
        const tsfm_chronos2_layer& y = a->layers[l];
        const float* src[11] = {y.time_norm, y.time_q, y.time_k, y.time_v, y.time_o, y.group_norm,
                                y.group_v, y.group_o, y.mlp_norm, y.mlp_wi, y.mlp_wo};
        const float* dst[11];
        for (int i = 0; i < 11; i++) {
            const size_t at = w_at[(size_t)l * 11 + i];
            if ((e = up(at, src[i], sizes[i])) != hipSuccess) return hip_fail(e, "host-to-device copy");
            dst[i] = reinterpret_cast<const float*>(base + at);
        }
        dev_layers[(size_t)l] = tsfm_chronos2_layer{dst[0], dst[1], dst[2], dst[3], dst[4], dst[5],
                                                    dst[6], dst[7], dst[8], dst[9], dst[10]};
    }
    float* x = reinterpret_cast<float*>(base + x_at);
    e = encode_on(a, x, reinterpret_cast<const uint8_t*>(base + kv_at), reinterpret_cast<const float*>(base + c_at),
                  reinterpret_cast<const float*>(base + s_at), dev_layers.data(),
                  reinterpret_cast<const float*>(base + fn_at), reinterpret_cast<float*>(base + scr_at), s);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "encoder launch");
    }
    if ((e = hipMemcpyAsync(a->x, x, x_n, hipMemcpyDeviceToHost, s)) != hipSuccess)
        return hip_fail(e, "device-to-host copy");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

// ---- Chronos-2 model forward: embedding, encoder stack, output head --------------------------------

namespace {

// Host buffers staged into the thread's device buffer: regions are planned first (src NULL = device
// scratch only), then the sources are uploaded in one pass.
struct Staging {
    struct Up { const void* src; size_t n, at; };
    Plan plan;
    std::vector<Up> ups;
    size_t add(const void* src, size_t n) {
        const size_t at = plan.take(n);
        if (src != nullptr && n > 0) ups.push_back({src, n, at});
        return at;
    }
    hipError_t upload(char* base, hipStream_t s) const {
        for (const Up& u : ups) {
            const hipError_t e = hipMemcpyAsync(base + u.at, u.src, u.n, hipMemcpyHostToDevice, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
};

// ResBlock.forward (src/core/resblock.zig:63-79) with ReLU: y = output(relu(hidden(x))) + residual(x),
// every linear with its bias. h: rows x hid, r: rows x out scratch.
hipError_t resblock_on(const tsfm_resblock& rb, const float* x, int rows, float* y, float* h, float* r, hipStream_t s) {
    hipError_t e = linear_on(x, rb.in, rb.hidden_w, rb.hid, rb.in, h, rb.hid, rows, tsfm::kEpiRelu, nullptr, s, rb.hidden_b);
    if (e == hipSuccess)
        e = linear_on(x, rb.in, rb.residual_w, rb.out, rb.in, r, rb.out, rows, tsfm::kEpiNone, nullptr, s, rb.residual_b);
    if (e == hipSuccess)
        e = linear_on(h, rb.hid, rb.output_w, rb.out, rb.hid, y, rb.out, rows, tsfm::kEpiResidual, r, s, rb.output_b);
    return e;
}

int validate_encode(const tsfm_chronos2_encode_args* a, bool needs_x) {
    if (a->batch < 0 || a->seq < 0 || a->n_layers < 0 || a->heads < 0 || a->d_ff < 0)
        return fail(TSFM_E_INVALID, "negative size");
    if (a->head_dim != 64) return fail(TSFM_E_UNSUPPORTED, "head_dim %d (supported: 64)", a->head_dim);
    if (a->d_model != a->heads * a->head_dim) return fail(TSFM_E_INVALID, "d_model != heads * head_dim");
    if ((int64_t)a->batch * a->seq == 0) return TSFM_OK;
    if (a->d_model == 0 || a->d_ff <= 0 || a->d_ff % 16)
        return fail(TSFM_E_UNSUPPORTED, "d_ff %d (supported: positive multiples of 16)", a->d_ff);
    if ((needs_x && (a->x == nullptr || a->key_valid == nullptr)) || a->rope_cos == nullptr ||
        a->rope_sin == nullptr || a->final_norm == nullptr || (a->n_layers > 0 && a->layers == nullptr))
        return fail(TSFM_E_INVALID, "x, key_valid, rope tables, final_norm and layers are required");
    for (int l = 0; l < a->n_layers; l++) {
        const tsfm_chronos2_layer& y = a->layers[l];
        const float* w[] = {y.time_norm, y.time_q, y.time_k, y.time_v, y.time_o, y.group_norm,
                            y.group_v, y.group_o, y.mlp_norm, y.mlp_wi, y.mlp_wo};
        for (const float* p : w)
            if (p == nullptr) return fail(TSFM_E_INVALID, "layer %d has a NULL weight", l);
    }
    if ((int64_t)a->batch * a->seq > 0x7fffffff / 4) return fail(TSFM_E_UNSUPPORTED, "too many tokens");
    return TSFM_OK;
}

int validate_resblock(const tsfm_resblock& rb, int in, int out, const char* what) {
    if (rb.in != in || (out > 0 && rb.out != out)) return fail(TSFM_E_INVALID, "%s: in/out do not match the model", what);
    if (rb.act != 0) return fail(TSFM_E_UNSUPPORTED, "%s: only the ReLU block (Chronos-2) runs here", what);
    if (rb.in <= 0 || rb.hid <= 0 || rb.out <= 0 || rb.in % 16 || rb.hid % 16 || rb.out % 4)
        return fail(TSFM_E_UNSUPPORTED, "%s: in and hid must be multiples of 16, out of 4", what);
    if (!rb.hidden_w || !rb.hidden_b || !rb.output_w || !rb.output_b || !rb.residual_w || !rb.residual_b)
        return fail(TSFM_E_INVALID, "%s: a weight or bias is NULL", what);
    return TSFM_OK;
}

// The forward on device buffers. x_buf: rows x d; kv: rows bytes; emb: rows x d; h: rows x hid_max;
// r: rows x out_max; enc: the encoder's scratch.
hipError_t forward_on(const tsfm_chronos2_forward_args* a, const tsfm_chronos2_encode_args& enc, const float* feats,
                      const float* fut_feats, const uint8_t* ctx_valid, const float* reg, float* raw, float* x_buf,
                      uint8_t* kv, float* emb, float* h, float* r, float* enc_scratch, hipStream_t s) {
    const int nb = enc.batch, d = enc.d_model, rows_ctx = nb * a->n_ctx, rows_fut = nb * a->n_out;
    float* emb_fut = emb + (int64_t)rows_ctx * d;
    hipError_t e = resblock_on(a->input_embed, feats, rows_ctx, emb, h, r, s);
    if (e == hipSuccess) e = resblock_on(a->input_embed, fut_feats, rows_fut, emb_fut, h, r, s);
    if (e == hipSuccess)
        e = tsfm::launch_assemble_sequence(emb, emb_fut, reg, ctx_valid, x_buf, kv, nb, a->n_ctx, a->n_out, d, s);
    if (e == hipSuccess)
        e = encode_on(&enc, x_buf, kv, enc.rope_cos, enc.rope_sin, enc.layers, enc.final_norm, enc_scratch, s);
    if (e == hipSuccess) e = tsfm::launch_gather_future(x_buf, emb, nb, a->n_ctx, a->n_out, d, s);
    if (e == hipSuccess) e = resblock_on(a->output_embed, emb, rows_fut, raw, h, r, s);
    return e;
}

}  // namespace

int tsfm_chronos2_forward(const tsfm_chronos2_forward_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (a->n_ctx < 0 || a->n_out < 0) return fail(TSFM_E_INVALID, "negative size");
    tsfm_chronos2_encode_args enc = a->enc;
    if (enc.seq != a->n_ctx + 1 + a->n_out) return fail(TSFM_E_INVALID, "enc.seq must be n_ctx + 1 + n_out");
    int rc = validate_encode(&enc, false);
    if (rc != TSFM_OK) return rc;
    if (enc.batch == 0) return TSFM_OK;
    if ((rc = validate_resblock(a->input_embed, a->input_embed.in, enc.d_model, "input_embed")) != TSFM_OK) return rc;
    if ((rc = validate_resblock(a->output_embed, enc.d_model, 0, "output_embed")) != TSFM_OK) return rc;
    if (a->feats == nullptr || a->fut_feats == nullptr || a->ctx_valid == nullptr || a->reg == nullptr || a->raw == nullptr)
        return fail(TSFM_E_INVALID, "feats, fut_feats, ctx_valid, reg and raw are required");
    rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    const int64_t nb = enc.batch, d = enc.d_model, rows = nb * enc.seq, F = enc.d_ff;
    const int64_t rows_ctx = nb * a->n_ctx, rows_fut = nb * a->n_out;
    const int64_t hid = std::max(a->input_embed.hid, a->output_embed.hid);
    const int64_t outw = std::max<int64_t>(d, a->output_embed.out);
    const size_t x_n = (size_t)(rows * d) * 4, kv_n = (size_t)rows, emb_n = (size_t)(rows * d) * 4;
    const size_t h_n = (size_t)(rows * hid) * 4, r_n = (size_t)(rows * outw) * 4;
    const size_t enc_n = encode_scratch_bytes(rows, d, F);
    const size_t raw_n = (size_t)(rows_fut * a->output_embed.out) * 4;
    const size_t planes_n = tsfm::proj_plane_bytes(rows, std::max({d, F, hid}), std::max({3 * d, F, hid, outw}));
    hipError_t e;
    if (enc.flags & TSFM_ATTN_DEVICE_PTRS) {
        bool ok = aligned(a->feats, 16) && aligned(a->fut_feats, 16) && aligned(a->reg, 16) && aligned(a->raw, 16) &&
                  aligned(enc.rope_cos, 16) && aligned(enc.rope_sin, 16) && aligned(enc.final_norm, 16);
        for (const tsfm_resblock* rb : {&a->input_embed, &a->output_embed})
            for (const float* p : {rb->hidden_w, rb->hidden_b, rb->output_w, rb->output_b, rb->residual_w, rb->residual_b})
                ok = ok && aligned(p, 16);
        for (int l = 0; l < enc.n_layers; l++) {
            const tsfm_chronos2_layer& y = enc.layers[l];
            for (const float* p : {y.time_norm, y.time_q, y.time_k, y.time_v, y.time_o, y.group_norm, y.group_v,
                                   y.group_o, y.mlp_norm, y.mlp_wi, y.mlp_wo})
                ok = ok && aligned(p, 16);
        }
        if (!ok) return fail(TSFM_E_UNSUPPORTED, "device pointers must be 16-byte aligned");
        hipStream_t s = static_cast<hipStream_t>(enc.stream);
        Plan plan;
        const size_t x_at = plan.take(x_n), kv_at = plan.take(kv_n), emb_at = plan.take(emb_n), h_at = plan.take(h_n),
                     r_at = plan.take(r_n), enc_at = plan.take(enc_n), part_at = plan.take(tsfm::kSplitWorkspaceBytes);
        const size_t planes_at = plan.take(planes_n);
        char* scratch = nullptr;
        bool owned = false;
        if ((e = tsfm::abi::scratch_acquire(s, tsfm::abi::kSlotChronos2Forward, plan.off, &scratch, &owned)) != hipSuccess)
            return hip_fail(e, "forward scratch allocation");
        tsfm::SplitWorkspace ws(reinterpret_cast<float*>(scratch + part_at));
        tsfm::PlaneWorkspace pws(scratch + planes_at, planes_n);
        e = forward_on(a, enc, a->feats, a->fut_feats, a->ctx_valid, a->reg, a->raw,
                       reinterpret_cast<float*>(scratch + x_at), reinterpret_cast<uint8_t*>(scratch + kv_at),
                       reinterpret_cast<float*>(scratch + emb_at), reinterpret_cast<float*>(scratch + h_at),
                       reinterpret_cast<float*>(scratch + r_at), reinterpret_cast<float*>(scratch + enc_at), s);
        const hipError_t f = owned ? hipFreeAsync(scratch, s) : hipSuccess;
        if (e != hipSuccess) return hip_fail(e, "forward launch");
        if (f != hipSuccess) return hip_fail(f, "forward scratch release");
        return TSFM_OK;
    }
    // Host pointers: stage every input and weight, run, copy the head's output back.
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    Staging st;
    const int64_t pin = a->input_embed.in;
    const size_t feats_at = st.add(a->feats, (size_t)(rows_ctx * pin) * 4);
    const size_t fut_at = st.add(a->fut_feats, (size_t)(rows_fut * pin) * 4);
    const size_t cv_at = st.add(a->ctx_valid, (size_t)rows_ctx);
    const size_t reg_at = st.add(a->reg, (size_t)d * 4);
    const size_t c_at = st.add(enc.rope_cos, (size_t)enc.seq * 32 * 4), s_at = st.add(enc.rope_sin, (size_t)enc.seq * 32 * 4);
    const size_t fn_at = st.add(enc.final_norm, (size_t)d * 4);
    auto stage_block = [&](const tsfm_resblock& rb, size_t at[6]) {
        at[0] = st.add(rb.hidden_w, (size_t)rb.hid * rb.in * 4);   at[1] = st.add(rb.hidden_b, (size_t)rb.hid * 4);
        at[2] = st.add(rb.output_w, (size_t)rb.out * rb.hid * 4);  at[3] = st.add(rb.output_b, (size_t)rb.out * 4);
        at[4] = st.add(rb.residual_w, (size_t)rb.out * rb.in * 4); at[5] = st.add(rb.residual_b, (size_t)rb.out * 4);
    };
    size_t in_at[6], out_at[6];
    stage_block(a->input_embed, in_at);
    stage_block(a->output_embed, out_at);
    const size_t dd = (size_t)(d * d) * 4, df = (size_t)(d * F) * 4, vn = (size_t)d * 4;
    const size_t sizes[11] = {vn, dd, dd, dd, dd, vn, dd, dd, vn, df, df};
    std::vector<size_t> w_at((size_t)enc.n_layers * 11);
    for (int l = 0; l < enc.n_layers; l++) {
        const tsfm_chronos2_layer& y = enc.layers[l];
        const float* src[11] = {y.time_norm, y.time_q, y.time_k, y.time_v, y.time_o, y.group_norm,
                                y.group_v, y.group_o, y.mlp_norm, y.mlp_wi, y.mlp_wo};
        for (int i = 0; i < 11; i++) w_at[(size_t)l * 11 + i] = st.add(src[i], sizes[i]);
    }
    const size_t x_at = st.add(nullptr, x_n), kv_at = st.add(nullptr, kv_n), emb_at = st.add(nullptr, emb_n);
    const size_t h_at = st.add(nullptr, h_n), r_at = st.add(nullptr, r_n), enc_at = st.add(nullptr, enc_n);
    const size_t raw_at = st.add(nullptr, raw_n), part_at = st.add(nullptr, tsfm::kSplitWorkspaceBytes);
    const size_t planes_at = st.add(nullptr, planes_n);
    rc = ensure_buf(ctx, st.plan.off);
    if (rc != TSFM_OK) return rc;
    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    tsfm::SplitWorkspace ws(reinterpret_cast<float*>(base + part_at));
    tsfm::PlaneWorkspace pws(base + planes_at, planes_n);
    if ((e = st.upload(base, s)) != hipSuccess) return hip_fail(e, "host-to-device copy");
    auto dp = [&](size_t at) { return reinterpret_cast<const float*>(base + at); };
    std::vector<tsfm_chronos2_layer> dev_layers((size_t)enc.n_layers);
    for (int l = 0; l < enc.n_layers; l++) {
        const size_t* w = &w_at[(size_t)l * 11];
        dev_layers[(size_t)l] = tsfm_chronos2_layer{dp(w[0]), dp(w[1]), dp(w[2]), dp(w[3]), dp(w[4]), dp(w[5]),
                                                    dp(w[6]), dp(w[7]), dp(w[8]), dp(w[9]), dp(w[10])};
    }
    tsfm_chronos2_forward_args da = *a;
    auto dev_block = [&](const tsfm_resblock& rb, const size_t at[6]) {
        tsfm_resblock o = rb;
        o.hidden_w = dp(at[0]); o.hidden_b = dp(at[1]); o.output_w = dp(at[2]); o.output_b = dp(at[3]);
        o.residual_w = dp(at[4]); o.residual_b = dp(at[5]);
        return o;
    };
    da.input_embed = dev_block(a->input_embed, in_at);
    da.output_embed = dev_block(a->output_embed, out_at);
    enc.rope_cos = dp(c_at); enc.rope_sin = dp(s_at); enc.final_norm = dp(fn_at); enc.layers = dev_layers.data();
    e = forward_on(&da, enc, dp(feats_at), dp(fut_at), reinterpret_cast<const uint8_t*>(base + cv_at), dp(reg_at),
                   reinterpret_cast<float*>(base + raw_at), reinterpret_cast<float*>(base + x_at),
                   reinterpret_cast<uint8_t*>(base + kv_at), reinterpret_cast<float*>(base + emb_at),
                   reinterpret_cast<float*>(base + h_at), reinterpret_cast<float*>(base + r_at),
                   reinterpret_cast<float*>(base + enc_at), s);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "forward launch");
    }
    if ((e = hipMemcpyAsync(a->raw, base + raw_at, raw_n, hipMemcpyDeviceToHost, s)) != hipSuccess)
        return hip_fail(e, "device-to-host copy");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

// ---- Chronos-Bolt model forward -------------------------------------------------------------------

namespace {

struct BoltDev {  // device-side pointers of one call
    const float *feats, *reg, *dec_start, *rel_table, *enc_final_norm, *dec_final_norm;
    const uint8_t* patch_valid;
    const int32_t* rel_bucket;
    const tsfm_bolt_enc_layer* enc;
    const tsfm_bolt_dec_layer* dec;
    tsfm_resblock ie, oe;
    float* raw;
};

// Scratch: x (rows x d), kv (rows bytes), emb (rows x d), xn (rows x d), q/k/v/ab (rows x inner
// each), hbuf (rows x max(d_ff, hid)), rbuf (rows x max(d, head out)), the bucket ids, and the
// cross-attention K/V of every decoder layer (2 x layers x rows x inner); the decoder reuses q/v/ab.
hipError_t bolt_forward_on(const tsfm_bolt_forward_args* a, const BoltDev& dv, char* scratch, const size_t* at,
                           hipStream_t s) {
    const int nb = a->batch, np = a->n_patch, seq = np + 1, d = a->d_model, inner = a->heads * a->head_dim;
    const int F = a->d_ff, R = nb * seq;
    float* x = reinterpret_cast<float*>(scratch + at[0]);
    uint8_t* kv = reinterpret_cast<uint8_t*>(scratch + at[1]);
    float* emb = reinterpret_cast<float*>(scratch + at[2]);
    float* xn = reinterpret_cast<float*>(scratch + at[3]);
    float* q = reinterpret_cast<float*>(scratch + at[4]);
    float* k = reinterpret_cast<float*>(scratch + at[5]);
    float* v = reinterpret_cast<float*>(scratch + at[6]);
    float* ab = reinterpret_cast<float*>(scratch + at[7]);
    float* hb = reinterpret_cast<float*>(scratch + at[8]);
    float* rb = reinterpret_cast<float*>(scratch + at[9]);
    hipError_t e = resblock_on(dv.ie, dv.feats, nb * np, emb, hb, rb, s);
    if (e == hipSuccess) e = tsfm::launch_assemble_sequence(emb, nullptr, dv.reg, dv.patch_valid, x, kv, nb, np, 0, d, s);
    // ---- encoder (Model.encode) ----
    // Each residual product also normalises its rows for what comes next (linear_norm_on): the o
    // projection for the FFN norm, wo for the next layer's attention norm or the final norm.
    if (e == hipSuccess)
        e = a->n_enc_layers > 0 ? tsfm::launch_rms_norm(x, d, xn, d, dv.enc[0].attn_norm, R, d, a->eps, s)
                                : tsfm::launch_rms_norm(x, d, x, d, dv.enc_final_norm, R, d, a->eps, s);
    for (int l = 0; l < a->n_enc_layers && e == hipSuccess; l++) {
        const tsfm_bolt_enc_layer& ly = dv.enc[l];
        const bool last = l + 1 == a->n_enc_layers;
        tsfm::ProjParams p{};
        p.x = xn; p.x_tok = d; p.w0 = ly.q; p.w1 = ly.k; p.w2 = ly.v; p.w_ld = d; p.alpha = 1.f;
        p.y0 = q; p.y1 = k; p.y2 = v; p.y0_tok = p.y1_tok = p.y2_tok = inner;
        p.tokens = R; p.seq = seq; p.d_in = d; p.width = inner; p.n_out = 3; p.out_dtype = TSFM_DTYPE_F32;
        if ((e = tsfm::launch_proj(p, s)) != hipSuccess) break;
        tsfm::Params ap{};
        ap.q = q; ap.k = k; ap.v = v; ap.o = ab;
        ap.q_tok = ap.k_tok = ap.v_tok = ap.o_tok = inner;
        ap.q_batch = ap.k_batch = ap.v_batch = ap.o_batch = (int64_t)seq * inner;
        ap.key_valid = kv; ap.kv_batch = seq;
        ap.rel_table = dv.rel_table; ap.rel_bucket = dv.rel_bucket; ap.rel_buckets = a->rel_buckets;
        ap.B = nb; ap.H = a->heads; ap.n_q = seq; ap.n_k = seq; ap.scale = 1.f;
        const int mask = a->keys_all_valid ? TSFM_MASK_FULL : TSFM_MASK_KEYS_ADDITIVE;  // Mask.pick(false, all, true)
        if ((e = tsfm::launch_attn_f32(ap, mask, tsfm::BIAS_REL, false, s)) != hipSuccess) break;
        if ((e = linear_norm_on(ab, inner, ly.o, d, inner, x, d, R, tsfm::kEpiResidual, x, ly.ffn_norm, xn, d, a->eps,
                                s)) != hipSuccess)
            break;
        if ((e = linear_on(xn, d, ly.wi, F, d, hb, F, R, tsfm::kEpiRelu, nullptr, s)) != hipSuccess) break;
        if ((e = linear_norm_on(hb, F, ly.wo, d, F, x, d, R, tsfm::kEpiResidual, x,
                                last ? dv.enc_final_norm : dv.enc[l + 1].attn_norm, last ? x : xn, d, a->eps, s)) !=
            hipSuccess)
            break;
    }
    // ---- the cross-attention K/V of every decoder layer from the encoder output: layers two at a
    //      time, one product of four outputs (fewer, fuller launches than one per layer) ----
    float* const ckv = reinterpret_cast<float*>(scratch + at[11]);
    const int64_t kv_n = (int64_t)R * inner;
    for (int l = 0; l < a->n_dec_layers && e == hipSuccess; l += 2) {
        const bool pair = l + 1 < a->n_dec_layers;
        tsfm::ProjParams p{};
        p.x = x; p.x_tok = d; p.w_ld = d; p.alpha = 1.f;
        p.w0 = dv.dec[l].cross_k; p.w1 = dv.dec[l].cross_v;
        p.y0 = ckv + (2 * l) * kv_n; p.y1 = ckv + (2 * l + 1) * kv_n;
        if (pair) {
            p.w2 = dv.dec[l + 1].cross_k; p.w3 = dv.dec[l + 1].cross_v;
            p.y2 = ckv + (2 * l + 2) * kv_n; p.y3 = ckv + (2 * l + 3) * kv_n;
        }
        p.y0_tok = p.y1_tok = p.y2_tok = p.y3_tok = inner;
        p.tokens = R; p.seq = seq; p.d_in = d; p.width = inner; p.n_out = pair ? 4 : 2; p.out_dtype = TSFM_DTYPE_F32;
        e = tsfm::launch_proj(p, s);
    }
    // ---- decoder (Model.decode): one token per series; y (nb x d) in emb ----
    float* y = emb;
    if (e == hipSuccess) e = tsfm::launch_broadcast_rows(dv.dec_start, y, nb, d, s);
    // With at most 16 series the decoder's products normalise their input rows as they load them
    // (the same bits as a norm launch first); otherwise each row norm is its own launch or is fused
    // into the producing product.
    const bool in_norm = tsfm::proj_fuses_input_norm(nb, d) && !unfused_norm_requested();
    if (e == hipSuccess && (!in_norm || a->n_dec_layers == 0))
        e = tsfm::launch_rms_norm(y, d, xn, d, a->n_dec_layers > 0 ? dv.dec[0].self_norm : dv.dec_final_norm, nb, d,
                                  a->eps, s);
    for (int l = 0; l < a->n_dec_layers && e == hipSuccess; l++) {
        const tsfm_bolt_dec_layer& ly = dv.dec[l];
        const bool last = l + 1 == a->n_dec_layers;
        // self-attention over the single decoder token: o(v(norm(y)))
        if (in_norm) {
            if ((e = linear_in_norm_on(y, d, ly.self_norm, a->eps, ly.self_v, inner, d, v, inner, nb, tsfm::kEpiNone,
                                       s)) != hipSuccess)
                break;
            if ((e = linear_on(v, inner, ly.self_o, d, inner, y, d, nb, tsfm::kEpiResidual, y, s)) != hipSuccess) break;
            if ((e = linear_in_norm_on(y, d, ly.cross_norm, a->eps, ly.cross_q, inner, d, q, inner, nb,
                                       tsfm::kEpiNone, s)) != hipSuccess)
                break;
        } else {
            // the o projection also normalises y for the cross-attention
            if ((e = linear_on(xn, d, ly.self_v, inner, d, v, inner, nb, tsfm::kEpiNone, nullptr, s)) != hipSuccess)
                break;
            if ((e = linear_norm_on(v, inner, ly.self_o, d, inner, y, d, nb, tsfm::kEpiResidual, y, ly.cross_norm, xn,
                                    d, a->eps, s)) != hipSuccess)
                break;
            if ((e = linear_on(xn, d, ly.cross_q, inner, d, q, inner, nb, tsfm::kEpiNone, nullptr, s)) != hipSuccess)
                break;
        }
        // cross-attention to the encoder output (its K/V computed above)
        tsfm::Params ap{};  // CrossJob.attend (:349-381): one query per (series, head), key mask, no scale
        ap.q = q; ap.k = ckv + (2 * l) * kv_n; ap.v = ckv + (2 * l + 1) * kv_n; ap.o = ab;
        ap.q_tok = inner; ap.q_batch = inner; ap.o_tok = inner; ap.o_batch = inner;
        ap.k_tok = ap.v_tok = inner; ap.k_batch = ap.v_batch = (int64_t)seq * inner;
        ap.key_valid = kv; ap.kv_batch = seq;
        ap.B = nb; ap.H = a->heads; ap.n_q = 1; ap.n_k = seq; ap.scale = 1.f;
        if ((e = tsfm::launch_attn_f32(ap, TSFM_MASK_KEYS_ADDITIVE, tsfm::BIAS_NONE, false, s)) != hipSuccess) break;
        // FFN; wo also normalises y for the next layer (or the final norm)
        if (in_norm) {
            if ((e = linear_on(ab, inner, ly.cross_o, d, inner, y, d, nb, tsfm::kEpiResidual, y, s)) != hipSuccess)
                break;
            if ((e = linear_in_norm_on(y, d, ly.ffn_norm, a->eps, ly.wi, F, d, hb, F, nb, tsfm::kEpiRelu, s)) !=
                hipSuccess)
                break;
            e = last ? linear_norm_on(hb, F, ly.wo, d, F, y, d, nb, tsfm::kEpiResidual, y, dv.dec_final_norm, xn, d,
                                      a->eps, s)
                     : linear_on(hb, F, ly.wo, d, F, y, d, nb, tsfm::kEpiResidual, y, s);
            if (e != hipSuccess) break;
        } else {
            if ((e = linear_norm_on(ab, inner, ly.cross_o, d, inner, y, d, nb, tsfm::kEpiResidual, y, ly.ffn_norm, xn,
                                    d, a->eps, s)) != hipSuccess)
                break;
            if ((e = linear_on(xn, d, ly.wi, F, d, hb, F, nb, tsfm::kEpiRelu, nullptr, s)) != hipSuccess) break;
            if ((e = linear_norm_on(hb, F, ly.wo, d, F, y, d, nb, tsfm::kEpiResidual, y,
                                    last ? dv.dec_final_norm : dv.dec[l + 1].self_norm, xn, d, a->eps, s)) !=
                hipSuccess)
                break;
        }
    }
    if (e == hipSuccess) e = resblock_on(dv.oe, xn, nb, dv.raw, hb, rb, s);
    return e;
}

}  // namespace

// Device copies of T5 bucket-id tables, one per (device, length, buckets, max distance), made on
// first use with a synchronous upload and kept until the process ends (a few KB each). Read-only
// after creation; the mutex guards the list.
static hipError_t cached_bucket_ids(const std::vector<int32_t>& ids, int64_t seq, int32_t buckets, int32_t max_distance,
                             const int32_t** out) {
    struct Entry {
        int device;
        int64_t seq;
        int32_t buckets, max_distance;
        int32_t* dev;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& c : cache)
        if (c.device == device && c.seq == seq && c.buckets == buckets && c.max_distance == max_distance) {
            *out = c.dev;
            return hipSuccess;
        }
    int32_t* dev = nullptr;
    if ((e = hipMalloc(reinterpret_cast<void**>(&dev), ids.size() * 4)) != hipSuccess) return e;
    if ((e = hipMemcpy(dev, ids.data(), ids.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) {
        (void)hipFree(dev);
        return e;
    }
    cache.push_back({device, seq, buckets, max_distance, dev});
    *out = dev;
    return hipSuccess;
}

int tsfm_bolt_forward(const tsfm_bolt_forward_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (a->batch < 0 || a->n_patch < 0 || a->n_enc_layers < 0 || a->n_dec_layers < 0 || a->heads < 0 || a->d_ff < 0)
        return fail(TSFM_E_INVALID, "negative size");
    if (a->head_dim != 64) return fail(TSFM_E_UNSUPPORTED, "head_dim %d (supported: 64)", a->head_dim);
    if (a->batch == 0) return TSFM_OK;
    const int64_t nb = a->batch, seq = (int64_t)a->n_patch + 1, d = a->d_model, inner = (int64_t)a->heads * 64;
    const int64_t F = a->d_ff, R = nb * seq;
    if (d <= 0 || d % 16 || F <= 0 || F % 16 || inner % 64 || inner == 0)
        return fail(TSFM_E_UNSUPPORTED, "d_model and d_ff must be positive multiples of 16");
    if (2 * seq - 1 > 2048) return fail(TSFM_E_UNSUPPORTED, "sequence too long for the T5 offset table");
    if (R > 0x7fffffff / 4) return fail(TSFM_E_UNSUPPORTED, "too many tokens");
    if (a->rel_buckets < 4 || a->rel_table == nullptr) return fail(TSFM_E_INVALID, "the T5 table is required");
    if (!a->feats || !a->patch_valid || !a->reg || !a->dec_start || !a->enc_final_norm || !a->dec_final_norm ||
        !a->raw || (a->n_enc_layers && !a->enc_layers) || (a->n_dec_layers && !a->dec_layers))
        return fail(TSFM_E_INVALID, "a required pointer is NULL");
    for (int l = 0; l < a->n_enc_layers; l++) {
        const tsfm_bolt_enc_layer& y = a->enc_layers[l];
        for (const float* p : {y.attn_norm, y.q, y.k, y.v, y.o, y.ffn_norm, y.wi, y.wo})
            if (p == nullptr) return fail(TSFM_E_INVALID, "encoder layer %d has a NULL weight", l);
    }
    for (int l = 0; l < a->n_dec_layers; l++) {
        const tsfm_bolt_dec_layer& y = a->dec_layers[l];
        for (const float* p : {y.self_norm, y.self_v, y.self_o, y.cross_norm, y.cross_q, y.cross_k, y.cross_v,
                               y.cross_o, y.ffn_norm, y.wi, y.wo})
            if (p == nullptr) return fail(TSFM_E_INVALID, "decoder layer %d has a NULL weight", l);
    }
    int rc;
    if ((rc = validate_resblock(a->input_embed, a->input_embed.in, (int)d, "input_embed")) != TSFM_OK) return rc;
    if ((rc = validate_resblock(a->output_embed, (int)d, 0, "output_embed")) != TSFM_OK) return rc;
    if ((rc = ensure_ready()) != TSFM_OK) return rc;
    // T5 bucket ids of key - query for the (seq, seq) self-attention (host, float32 log as the reference).
    std::vector<int32_t> buckets((size_t)(2 * seq - 1));
    if ((rc = tsfm_t5_bucket_table(buckets.data(), (int32_t)seq, (int32_t)seq, (uint32_t)a->rel_buckets,
                                   (uint32_t)a->rel_max_distance)) != TSFM_OK)
        return rc;
    const int64_t hid = std::max(std::max<int64_t>(a->input_embed.hid, a->output_embed.hid), F);
    const int64_t rw = std::max<int64_t>(d, a->output_embed.out);
    const size_t sz[12] = {(size_t)(R * d) * 4, (size_t)R, (size_t)(R * d) * 4, (size_t)(R * d) * 4,
                           (size_t)(R * inner) * 4, (size_t)(R * inner) * 4, (size_t)(R * inner) * 4,
                           (size_t)(R * inner) * 4, (size_t)(R * hid) * 4, (size_t)(R * rw) * 4,
                           buckets.size() * 4, (size_t)(2 * a->n_dec_layers * R * inner) * 4};
    hipError_t e;
    if (a->flags & TSFM_ATTN_DEVICE_PTRS) {
        hipStream_t s = static_cast<hipStream_t>(a->stream);
        Plan plan;
        size_t at[12];
        for (int i = 0; i < 12; i++) at[i] = plan.take(sz[i]);
        const size_t part_at = plan.take(tsfm::kSplitWorkspaceBytes);
        // The bucket ids live on the device once per (length, buckets, max distance): a per-call
        // upload from pageable memory would make the host wait for the stream to drain before it
        // could queue the forward's launches.
        const int32_t* ids = nullptr;
        if ((e = cached_bucket_ids(buckets, seq, a->rel_buckets, a->rel_max_distance, &ids)) != hipSuccess)
            return hip_fail(e, "bucket id upload");
        char* scratch = nullptr;
        bool owned = false;
        if ((e = tsfm::abi::scratch_acquire(s, tsfm::abi::kSlotBoltForward, plan.off, &scratch, &owned)) != hipSuccess)
            return hip_fail(e, "forward scratch allocation");
        BoltDev dv{a->feats, a->reg, a->dec_start, a->rel_table, a->enc_final_norm, a->dec_final_norm,
                   a->patch_valid, ids, a->enc_layers, a->dec_layers, a->input_embed, a->output_embed, a->raw};
        {
            tsfm::SplitWorkspace ws(reinterpret_cast<float*>(scratch + part_at));
            e = bolt_forward_on(a, dv, scratch, at, s);
        }
        const hipError_t f = owned ? hipFreeAsync(scratch, s) : hipSuccess;
        if (e != hipSuccess) return hip_fail(e, "forward launch");
        if (f != hipSuccess) return hip_fail(f, "forward scratch release");
        return TSFM_OK;
    }
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    Staging st;
    size_t at[12];
    for (int i = 0; i < 10; i++) at[i] = st.add(nullptr, sz[i]);
    at[10] = st.add(buckets.data(), sz[10]);
    at[11] = st.add(nullptr, sz[11]);
    const int64_t pin = a->input_embed.in;
    const size_t feats_at = st.add(a->feats, (size_t)(nb * a->n_patch * pin) * 4);
    const size_t pv_at = st.add(a->patch_valid, (size_t)(nb * a->n_patch));
    const size_t reg_at = st.add(a->reg, (size_t)d * 4), ds_at = st.add(a->dec_start, (size_t)d * 4);
    const size_t rt_at = st.add(a->rel_table, (size_t)a->rel_buckets * a->heads * 4);
    const size_t ef_at = st.add(a->enc_final_norm, (size_t)d * 4), df_at = st.add(a->dec_final_norm, (size_t)d * 4);
    const size_t raw_at = st.add(nullptr, (size_t)(nb * a->output_embed.out) * 4);
    const size_t part_at = st.add(nullptr, tsfm::kSplitWorkspaceBytes);
    auto stage_block = [&](const tsfm_resblock& rb, size_t o[6]) {
        o[0] = st.add(rb.hidden_w, (size_t)rb.hid * rb.in * 4);   o[1] = st.add(rb.hidden_b, (size_t)rb.hid * 4);
        o[2] = st.add(rb.output_w, (size_t)rb.out * rb.hid * 4);  o[3] = st.add(rb.output_b, (size_t)rb.out * 4);
        o[4] = st.add(rb.residual_w, (size_t)rb.out * rb.in * 4); o[5] = st.add(rb.residual_b, (size_t)rb.out * 4);
    };
    size_t ie_at[6], oe_at[6];
    stage_block(a->input_embed, ie_at);
    stage_block(a->output_embed, oe_at);
    const size_t vd = (size_t)d * 4, di = (size_t)(d * inner) * 4, df = (size_t)(d * F) * 4;
    const size_t enc_sz[8] = {vd, di, di, di, di, vd, df, df};
    const size_t dec_sz[11] = {vd, di, di, vd, di, di, di, di, vd, df, df};
    std::vector<size_t> ew((size_t)a->n_enc_layers * 8), dw((size_t)a->n_dec_layers * 11);
    for (int l = 0; l < a->n_enc_layers; l++) {
        const tsfm_bolt_enc_layer& y = a->enc_layers[l];
        const float* src[8] = {y.attn_norm, y.q, y.k, y.v, y.o, y.ffn_norm, y.wi, y.wo};
        for (int i = 0; i < 8; i++) ew[(size_t)l * 8 + i] = st.add(src[i], enc_sz[i]);
    }
    for (int l = 0; l < a->n_dec_layers; l++) {
        const tsfm_bolt_dec_layer& y = a->dec_layers[l];
        const float* src[11] = {y.self_norm, y.self_v, y.self_o, y.cross_norm, y.cross_q, y.cross_k, y.cross_v,
                                y.cross_o, y.ffn_norm, y.wi, y.wo};
        for (int i = 0; i < 11; i++) dw[(size_t)l * 11 + i] = st.add(src[i], dec_sz[i]);
    }
    if ((rc = ensure_buf(ctx, st.plan.off)) != TSFM_OK) return rc;
    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    tsfm::SplitWorkspace ws(reinterpret_cast<float*>(base + part_at));
    if ((e = st.upload(base, s)) != hipSuccess) return hip_fail(e, "host-to-device copy");
    auto dp = [&](size_t off) { return reinterpret_cast<const float*>(base + off); };
    std::vector<tsfm_bolt_enc_layer> el((size_t)a->n_enc_layers);
    std::vector<tsfm_bolt_dec_layer> dl((size_t)a->n_dec_layers);
    for (int l = 0; l < a->n_enc_layers; l++) {
        const size_t* w = &ew[(size_t)l * 8];
        el[(size_t)l] = tsfm_bolt_enc_layer{dp(w[0]), dp(w[1]), dp(w[2]), dp(w[3]), dp(w[4]), dp(w[5]), dp(w[6]), dp(w[7])};
    }
    for (int l = 0; l < a->n_dec_layers; l++) {
        const size_t* w = &dw[(size_t)l * 11];
        dl[(size_t)l] = tsfm_bolt_dec_layer{dp(w[0]), dp(w[1]), dp(w[2]), dp(w[3]), dp(w[4]), dp(w[5]),
                                            dp(w[6]), dp(w[7]), dp(w[8]), dp(w[9]), dp(w[10])};
    }
    auto dev_block = [&](const tsfm_resblock& rb, const size_t o[6]) {
        tsfm_resblock r = rb;
        r.hidden_w = dp(o[0]); r.hidden_b = dp(o[1]); r.output_w = dp(o[2]); r.output_b = dp(o[3]);
        r.residual_w = dp(o[4]); r.residual_b = dp(o[5]);
        return r;
    };
    BoltDev dv{dp(feats_at), dp(reg_at), dp(ds_at), dp(rt_at), dp(ef_at), dp(df_at),
               reinterpret_cast<const uint8_t*>(base + pv_at), reinterpret_cast<const int32_t*>(base + at[10]),
               el.data(), dl.data(), dev_block(a->input_embed, ie_at), dev_block(a->output_embed, oe_at),
               reinterpret_cast<float*>(base + raw_at)};
    e = bolt_forward_on(a, dv, base, at, s);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "forward launch");
    }
    if ((e = hipMemcpyAsync(a->raw, base + raw_at, (size_t)(nb * a->output_embed.out) * 4, hipMemcpyDeviceToHost, s)) !=
        hipSuccess)
        return hip_fail(e, "device-to-host copy");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

int tsfm_bolt_forecast(const tsfm_bolt_forecast_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (!(a->model.flags & TSFM_ATTN_DEVICE_PTRS))
        return fail(TSFM_E_UNSUPPORTED, "the forecast takes device weights (TSFM_ATTN_DEVICE_PTRS; TSFM_FORECAST_HOST_IO "
                                        "for host inputs and outputs); host callers may use tsfm_bolt_forward");
    if (a->len <= 0 || a->patch <= 0 || a->ctx == nullptr || a->out == nullptr || a->stride < 0 || a->offset < 0)
        return fail(TSFM_E_INVALID, "bad context description");
    if (a->model.flags & TSFM_FORECAST_HOST_IO) {
        const int64_t nb = a->model.batch, per = a->model.output_embed.out;
        if (nb < 0 || per < 0) return fail(TSFM_E_INVALID, "negative size");
        if (nb == 0) return TSFM_OK;
        tsfm_bolt_forecast_args d = *a;
        d.model.flags &= ~TSFM_FORECAST_HOST_IO;
        const size_t ctx_n = (size_t)((nb - 1) * a->stride + a->offset + a->len) * 4;
        return tsfm::abi::run_host_io({{a->ctx, ctx_n, reinterpret_cast<const void**>(&d.ctx)}},
                                      {{a->out, (size_t)(nb * per) * 4, const_cast<const void**>(reinterpret_cast<void**>(&d.out))}},
                                      [&](hipStream_t s) {
                                          d.model.stream = s;
                                          return tsfm_bolt_forecast(&d);
                                      });
    }
    const int32_t pad = (a->patch - a->len % a->patch) % a->patch, n_patch = (a->len + pad) / a->patch;
    if (a->model.n_patch != n_patch) return fail(TSFM_E_INVALID, "model.n_patch must be ceil(len / patch)");
    if (a->model.input_embed.in != 2 * a->patch) return fail(TSFM_E_INVALID, "input_embed.in must be 2 * patch");
    const int64_t nb = a->model.batch;
    if (nb < 0) return fail(TSFM_E_INVALID, "negative size");
    if (nb == 0) return TSFM_OK;
    if (!aligned(a->out, 16)) return fail(TSFM_E_UNSUPPORTED, "device pointers must be 16-byte aligned");
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(a->model.stream);
    const int64_t per = a->model.output_embed.out;
    Plan plan;
    const size_t f_at = plan.take((size_t)(nb * n_patch * 2 * a->patch) * 4), pv_at = plan.take((size_t)(nb * n_patch));
    const size_t lo_at = plan.take((size_t)nb * 4), sc_at = plan.take((size_t)nb * 4), raw_at = plan.take((size_t)(nb * per) * 4);
    char* buf = nullptr;
    bool owned = false;
    hipError_t e;
    if ((e = tsfm::abi::scratch_acquire(s, tsfm::abi::kSlotBoltForecast, plan.off, &buf, &owned)) != hipSuccess)
        return hip_fail(e, "forecast scratch allocation");
    float* feats = reinterpret_cast<float*>(buf + f_at);
    uint8_t* pv = reinterpret_cast<uint8_t*>(buf + pv_at);
    float* lo = reinterpret_cast<float*>(buf + lo_at);
    float* sc = reinterpret_cast<float*>(buf + sc_at);
    float* raw = reinterpret_cast<float*>(buf + raw_at);
    e = tsfm::launch_bolt_prepare(a->ctx, a->stride, a->offset, a->len, a->patch, n_patch, pad, a->norm_eps, feats, pv, lo,
                                  sc, (int)nb, s);
    if (e == hipSuccess) {
        tsfm_bolt_forward_args m = a->model;
        m.feats = feats; m.patch_valid = pv; m.raw = raw;
        m.keys_all_valid = 0;  // validity is only known on the device: the additive mask, exact either way
        rc = tsfm_bolt_forward(&m);
        if (rc != TSFM_OK) {
            if (owned) (void)hipFreeAsync(buf, s);
            return rc;
        }
        e = tsfm::launch_bolt_finish(raw, lo, sc, a->out, (int)nb, (int)per, s);
    }
    const hipError_t f = owned ? hipFreeAsync(buf, s) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "forecast launch");
    if (f != hipSuccess) return hip_fail(f, "forecast scratch release");
    return TSFM_OK;
}

int tsfm_chronos2_forecast(const tsfm_chronos2_forecast_args* a) {
    if (a == nullptr) return fail(TSFM_E_INVALID, "args is NULL");
    if (!(a->model.enc.flags & TSFM_ATTN_DEVICE_PTRS))
        return fail(TSFM_E_UNSUPPORTED, "the forecast takes device weights (TSFM_ATTN_DEVICE_PTRS; TSFM_FORECAST_HOST_IO "
                                        "for host inputs and outputs); host callers may use tsfm_chronos2_forward");
    const int32_t ps = a->model.input_embed.in / 3;
    if (ps <= 0 || a->model.input_embed.in != 3 * ps) return fail(TSFM_E_INVALID, "input_embed.in must be 3 * patch");
    if (a->len <= 0 || a->horizon <= 0 || a->inputs == nullptr || a->out == nullptr || a->stride < 0 || a->start < 0 ||
        !(a->time_scale != 0.f))
        return fail(TSFM_E_INVALID, "bad context description");
    const int32_t pad = (ps - a->len % ps) % ps, n_ctx = (a->len + pad) / ps, n_out = (a->horizon + ps - 1) / ps;
    if (a->model.n_ctx != n_ctx) return fail(TSFM_E_INVALID, "model.n_ctx must be ceil(len / patch)");
    if (a->model.n_out != n_out) return fail(TSFM_E_INVALID, "model.n_out must be ceil(horizon / patch)");
    const int32_t per = a->model.output_embed.out;
    if (per <= 0 || per % ps) return fail(TSFM_E_INVALID, "output_embed.out must be q * patch");
    const int64_t nb = a->model.enc.batch;
    if (nb < 0) return fail(TSFM_E_INVALID, "negative size");
    if (nb == 0) return TSFM_OK;
    if (a->model.enc.flags & TSFM_FORECAST_HOST_IO) {
        tsfm_chronos2_forecast_args d = *a;
        d.model.enc.flags &= ~TSFM_FORECAST_HOST_IO;
        const size_t in_n = (size_t)((nb - 1) * a->stride + a->start + a->len) * 4;
        const size_t out_n = (size_t)(nb * a->horizon * (per / ps)) * 4;
        return tsfm::abi::run_host_io({{a->inputs, in_n, reinterpret_cast<const void**>(&d.inputs)}},
                                      {{a->out, out_n, const_cast<const void**>(reinterpret_cast<void**>(&d.out))}},
                                      [&](hipStream_t s) {
                                          d.model.enc.stream = s;
                                          return tsfm_chronos2_forecast(&d);
                                      });
    }
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(a->model.enc.stream);
    Plan plan;
    const size_t f_at = plan.take((size_t)(nb * n_ctx * 3 * ps) * 4), ff_at = plan.take((size_t)(nb * n_out * 3 * ps) * 4);
    const size_t cv_at = plan.take((size_t)(nb * n_ctx)), lo_at = plan.take((size_t)nb * 4);
    const size_t sc_at = plan.take((size_t)nb * 4), raw_at = plan.take((size_t)(nb * n_out * per) * 4);
    char* buf = nullptr;
    bool owned = false;
    hipError_t e;
    if ((e = tsfm::abi::scratch_acquire(s, tsfm::abi::kSlotChronos2Forecast, plan.off, &buf, &owned)) != hipSuccess)
        return hip_fail(e, "forecast scratch allocation");
    float* feats = reinterpret_cast<float*>(buf + f_at);
    float* fut = reinterpret_cast<float*>(buf + ff_at);
    uint8_t* cv = reinterpret_cast<uint8_t*>(buf + cv_at);
    float* lo = reinterpret_cast<float*>(buf + lo_at);
    float* sc = reinterpret_cast<float*>(buf + sc_at);
    float* raw = reinterpret_cast<float*>(buf + raw_at);
    e = tsfm::launch_chronos2_prepare(a->inputs, a->stride, a->start, a->len, ps, n_ctx, n_out, pad, a->time_scale,
                                      a->arcsinh ? 1 : 0, feats, fut, cv, lo, sc, (int)nb, s);
    if (e == hipSuccess) {
        tsfm_chronos2_forward_args m = a->model;
        m.feats = feats; m.fut_feats = fut; m.ctx_valid = cv; m.raw = raw;
        m.enc.keys_all_valid = 0;  // validity is only known on the device: the additive mask, exact either way
        rc = tsfm_chronos2_forward(&m);
        if (rc != TSFM_OK) {
            if (owned) (void)hipFreeAsync(buf, s);
            return rc;
        }
        e = tsfm::launch_chronos2_finish(raw, lo, sc, a->out, (int)nb, n_out, per / ps, ps, a->horizon,
                                         a->arcsinh ? 1 : 0, s);
    }
    const hipError_t f = owned ? hipFreeAsync(buf, s) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "forecast launch");
    if (f != hipSuccess) return hip_fail(f, "forecast scratch release");
    return TSFM_OK;
}

// ---- the reference backend's GEMM seam ------------------------------------------------------------

void* tsfm_weight_register(const float* data, size_t len) {
    if (len == 0 || data == nullptr || ensure_ready() != TSFM_OK) return nullptr;
    void* dev = nullptr;
    if (hipSetDevice(g_device) != hipSuccess || hipMalloc(&dev, len * sizeof(float)) != hipSuccess || dev == nullptr) {
        fail(TSFM_E_DEVICE, "weight allocation of %zu floats failed", len);
        return nullptr;
    }
    if (hipMemcpy(dev, data, len * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(dev);
        fail(TSFM_E_DEVICE, "weight upload failed");
        return nullptr;
    }
    return dev;
}

void tsfm_weight_release(void* handle) {
    if (handle != nullptr) (void)hipFree(handle);
}

int tsfm_sgemm_nt(int m, int n, int k, float alpha, const float* A, int lda, const float* B, int ldb, float* C, int ldc,
                  void* b_buf) {
    if (m <= 0 || n <= 0 || k <= 0) return fail(TSFM_E_INVALID, "empty or negative product %d x %d x %d", m, n, k);
    if (A == nullptr || C == nullptr || (B == nullptr && b_buf == nullptr)) return fail(TSFM_E_INVALID, "NULL operand");
    if (lda < k || ldb < k || ldc < n) return fail(TSFM_E_INVALID, "leading dimension shorter than the row");
    if (k % 16 || n % 4 || lda % 4 || ldb % 4 || ldc % 4)
        return fail(TSFM_E_UNSUPPORTED, "k must be a multiple of 16, n and the leading dimensions of 4");
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    const size_t a_n = ((size_t)(m - 1) * lda + k) * 4, b_n = b_buf ? 0 : ((size_t)(n - 1) * ldb + k) * 4;
    const size_t c_n = ((size_t)(m - 1) * ldc + n) * 4;
    Plan plan;
    const size_t a_at = plan.take(a_n), b_at = plan.take(b_n), c_at = plan.take(c_n);
    const size_t part_at = plan.take(tsfm::kSplitWorkspaceBytes);
    rc = ensure_buf(ctx, plan.off);
    if (rc != TSFM_OK) return rc;
    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    tsfm::SplitWorkspace ws(reinterpret_cast<float*>(base + part_at));
    hipError_t e;
    if ((e = hipMemcpyAsync(base + a_at, A, a_n, hipMemcpyHostToDevice, s)) != hipSuccess)
        return hip_fail(e, "host-to-device copy");
    if (b_n && (e = hipMemcpyAsync(base + b_at, B, b_n, hipMemcpyHostToDevice, s)) != hipSuccess)
        return hip_fail(e, "host-to-device copy");
    tsfm::ProjParams p{};
    p.x = reinterpret_cast<const float*>(base + a_at); p.x_tok = lda;
    p.w0 = b_buf ? static_cast<const float*>(b_buf) : reinterpret_cast<const float*>(base + b_at);
    p.w_ld = ldb; p.alpha = alpha; p.epi = tsfm::kEpiNone;
    p.y0 = base + c_at; p.y0_tok = ldc;
    p.tokens = m; p.seq = m; p.d_in = k; p.width = n; p.n_out = 1; p.out_dtype = TSFM_DTYPE_F32;
    if ((e = tsfm::launch_proj(p, s)) != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "GEMM launch");
    }
    if ((e = copy_rows_d2h(C, base + c_at, 1, m, 0, (int64_t)ldc * 4, (int64_t)n * 4, s)) != hipSuccess)
        return hip_fail(e, "device-to-host copy");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

int tsfm_sgemm_nn(int m, int n, int k, const float* A, int lda, const float* B, int ldb, float* C, int ldc,
                  void* b_buf) {
    if (m <= 0 || n <= 0 || k <= 0) return fail(TSFM_E_INVALID, "empty or negative product %d x %d x %d", m, n, k);
    if (A == nullptr || C == nullptr || (B == nullptr && b_buf == nullptr)) return fail(TSFM_E_INVALID, "NULL operand");
    if (lda < k || ldb < n || ldc < n) return fail(TSFM_E_INVALID, "leading dimension shorter than the row");
    if (k % 16 || n % 4 || lda % 4 || ldc % 4)
        return fail(TSFM_E_UNSUPPORTED, "k must be a multiple of 16, n, lda and ldc of 4");
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    // B [k][ldb] is transposed on the device to B^T [n][k], and the product runs as A (B^T)^T on the
    // projection kernel, like tsfm_sgemm_nt.
    const size_t a_n = ((size_t)(m - 1) * lda + k) * 4, b_n = b_buf ? 0 : ((size_t)(k - 1) * ldb + n) * 4;
    const size_t bt_n = (size_t)n * k * 4, c_n = ((size_t)(m - 1) * ldc + n) * 4;
    Plan plan;
    const size_t a_at = plan.take(a_n), b_at = plan.take(b_n), bt_at = plan.take(bt_n), c_at = plan.take(c_n);
    const size_t part_at = plan.take(tsfm::kSplitWorkspaceBytes);
    rc = ensure_buf(ctx, plan.off);
    if (rc != TSFM_OK) return rc;
    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    tsfm::SplitWorkspace ws(reinterpret_cast<float*>(base + part_at));
    hipError_t e;
    if ((e = hipMemcpyAsync(base + a_at, A, a_n, hipMemcpyHostToDevice, s)) != hipSuccess)
        return hip_fail(e, "host-to-device copy");
    if (b_n && (e = hipMemcpyAsync(base + b_at, B, b_n, hipMemcpyHostToDevice, s)) != hipSuccess)
        return hip_fail(e, "host-to-device copy");
    const float* bd = b_buf ? static_cast<const float*>(b_buf) : reinterpret_cast<const float*>(base + b_at);
    float* bt = reinterpret_cast<float*>(base + bt_at);
    tsfm::ProjParams p{};
    p.x = reinterpret_cast<const float*>(base + a_at); p.x_tok = lda;
    p.w0 = bt; p.w_ld = k; p.alpha = 1.f; p.epi = tsfm::kEpiNone;
    p.y0 = base + c_at; p.y0_tok = ldc;
    p.tokens = m; p.seq = m; p.d_in = k; p.width = n; p.n_out = 1; p.out_dtype = TSFM_DTYPE_F32;
    if ((e = tsfm::launch_transpose_f32(bd, ldb, bt, k, k, n, s)) != hipSuccess ||
        (e = tsfm::launch_proj(p, s)) != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "GEMM launch");
    }
    if ((e = copy_rows_d2h(C, base + c_at, 1, m, 0, (int64_t)ldc * 4, (int64_t)n * 4, s)) != hipSuccess)
        return hip_fail(e, "device-to-host copy");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

// ---- KV cache ------------------------------------------------------------------------------------

struct tsfm_kv_cache {
    int32_t dtype, B, H, D, cap, len;
    void* k;
    void* v;
};

int tsfm_kv_create(tsfm_kv_cache** out, int32_t dtype, int32_t batch, int32_t heads, int32_t head_dim,
                   int32_t capacity) {
    if (out == nullptr) return fail(TSFM_E_INVALID, "out is NULL");
    *out = nullptr;
    if (dtype != TSFM_DTYPE_BF16 && dtype != TSFM_DTYPE_F16) return fail(TSFM_E_UNSUPPORTED, "KV cache is bf16/f16 only");
    if (head_dim != 64) return fail(TSFM_E_UNSUPPORTED, "head_dim %d (supported: 64)", head_dim);
    if (batch <= 0 || heads <= 0 || capacity <= 0) return fail(TSFM_E_INVALID, "bad cache shape");
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    // Whole 64-key tiles: the decode kernel reads every row of the tiles it touches.
    const int32_t cap = (capacity + 63) / 64 * 64;
    const size_t bytes = (size_t)batch * heads * cap * head_dim * 2;
    tsfm_kv_cache* c = new tsfm_kv_cache{dtype, batch, heads, head_dim, cap, 0, nullptr, nullptr};
    if (hipSetDevice(g_device) != hipSuccess || hipMalloc(&c->k, bytes) != hipSuccess ||
        hipMalloc(&c->v, bytes) != hipSuccess) {
        if (c->k) (void)hipFree(c->k);
        delete c;
        return fail(TSFM_E_DEVICE, "KV cache allocation of 2 x %zu bytes failed", bytes);
    }
    // Rows past the length are read (and masked) by the decode kernel: keep them finite.
    if (hipMemset(c->k, 0, bytes) != hipSuccess || hipMemset(c->v, 0, bytes) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(c->k);
        (void)hipFree(c->v);
        delete c;
        return fail(TSFM_E_DEVICE, "KV cache initialisation failed");
    }
    *out = c;
    return TSFM_OK;
}

int tsfm_kv_free(tsfm_kv_cache* c) {
    if (c == nullptr) return TSFM_OK;
    (void)hipDeviceSynchronize();
    if (c->k) (void)hipFree(c->k);
    if (c->v) (void)hipFree(c->v);
    delete c;
    return TSFM_OK;
}

int tsfm_kv_reset(tsfm_kv_cache* c) {
    if (c == nullptr) return fail(TSFM_E_INVALID, "cache is NULL");
    c->len = 0;
    return TSFM_OK;
}

int tsfm_kv_truncate(tsfm_kv_cache* c, int32_t len) {
    if (c == nullptr) return fail(TSFM_E_INVALID, "cache is NULL");
    if (len < 0 || len > c->len) return fail(TSFM_E_INVALID, "truncate to %d outside [0, %d]", len, c->len);
    c->len = len;
    return TSFM_OK;
}

int32_t tsfm_kv_len(const tsfm_kv_cache* c) { return c == nullptr ? 0 : c->len; }

int tsfm_kv_append(tsfm_kv_cache* c, const void* k, int64_t k_tok, int64_t k_batch, const void* v, int64_t v_tok,
                   int64_t v_batch, int32_t n_new, uint32_t flags, void* stream) {
    if (c == nullptr || k == nullptr || v == nullptr) return fail(TSFM_E_INVALID, "NULL argument");
    if (n_new < 0 || k_tok < 0 || k_batch < 0 || v_tok < 0 || v_batch < 0) return fail(TSFM_E_INVALID, "negative size");
    if (n_new == 0) return TSFM_OK;
    if ((int64_t)c->len + n_new > c->cap)
        return fail(TSFM_E_INVALID, "append of %d exceeds capacity %d (len %d)", n_new, c->cap, c->len);
    if (k_tok % 8 || k_batch % 8 || v_tok % 8 || v_batch % 8) return fail(TSFM_E_UNSUPPORTED, "strides must be multiples of 16 bytes");
    if (span_checked(c->B, n_new, k_tok, k_batch, (int64_t)c->H * c->D) < 0 ||
        span_checked(c->B, n_new, v_tok, v_batch, (int64_t)c->H * c->D) < 0)
        return fail(TSFM_E_UNSUPPORTED, "a k/v view spans more than 2^46 elements");
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    tsfm::KvLayout L{c->k, c->v, c->B, c->H, c->cap};
    const bool bf16 = c->dtype == TSFM_DTYPE_BF16;
    hipError_t e;
    if (flags & TSFM_ATTN_DEVICE_PTRS) {
        if (!aligned(k, 16) || !aligned(v, 16)) return fail(TSFM_E_UNSUPPORTED, "device k/v must be 16-byte aligned");
        e = tsfm::launch_kv_append(L, bf16, k, k_tok, k_batch, v, v_tok, v_batch, c->len, n_new,
                                   static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail(e, "KV append launch");
    } else {
        const int64_t row = (int64_t)c->H * c->D;
        const size_t k_n = span(c->B, n_new, k_tok, k_batch, row) * 2, v_n = span(c->B, n_new, v_tok, v_batch, row) * 2;
        Plan plan;
        const size_t k_at = plan.take(k_n), v_at = plan.take(v_n);
        rc = ensure_buf(ctx, plan.off);
        if (rc != TSFM_OK) return rc;
        char* base = static_cast<char*>(ctx->buf);
        hipStream_t s = ctx->stream;
        if ((e = hipMemcpyAsync(base + k_at, k, k_n, hipMemcpyHostToDevice, s)) != hipSuccess ||
            (e = hipMemcpyAsync(base + v_at, v, v_n, hipMemcpyHostToDevice, s)) != hipSuccess)
            return hip_fail(e, "host-to-device copy");
        e = tsfm::launch_kv_append(L, bf16, base + k_at, k_tok, k_batch, base + v_at, v_tok, v_batch, c->len, n_new, s);
        if (e != hipSuccess) return hip_fail(e, "KV append launch");
        if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    }
    c->len += n_new;
    return TSFM_OK;
}

int tsfm_kv_attend(tsfm_kv_cache* c, const void* q, int64_t q_tok, int64_t q_batch, void* o, int64_t o_tok,
                   int64_t o_batch, int32_t n_q, int32_t q_pos0, float scale, uint32_t flags, void* stream) {
    if (c == nullptr || q == nullptr || o == nullptr) return fail(TSFM_E_INVALID, "NULL argument");
    if (n_q < 0 || q_pos0 < 0 || q_tok < 0 || q_batch < 0 || o_tok < 0 || o_batch < 0)
        return fail(TSFM_E_INVALID, "negative size");
    if (n_q == 0) return TSFM_OK;
    if ((int64_t)q_pos0 + n_q > c->len)
        return fail(TSFM_E_INVALID, "queries [%d, %lld) beyond cache length %d", q_pos0, (long long)q_pos0 + n_q, c->len);
    if (q_tok % 8 || q_batch % 8 || o_tok % 8 || o_batch % 8) return fail(TSFM_E_UNSUPPORTED, "strides must be multiples of 16 bytes");
    const int64_t row = (int64_t)c->H * c->D;
    if (o_tok < row && n_q > 1) return fail(TSFM_E_INVALID, "o token stride smaller than heads * head_dim");
    if (span_checked(c->B, n_q, q_tok, q_batch, row) < 0 || span_checked(c->B, n_q, o_tok, o_batch, row) < 0)
        return fail(TSFM_E_UNSUPPORTED, "a q/o view spans more than 2^46 elements");
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    ThreadCtx* ctx = thread_ctx();
    if (ctx == nullptr) return fail(TSFM_E_DEVICE, "cannot create the thread's HIP stream");
    tsfm::KvLayout L{c->k, c->v, c->B, c->H, c->cap};
    const bool bf16 = c->dtype == TSFM_DTYPE_BF16;
    const int32_t n_k = q_pos0 + n_q;
    hipError_t e;
    if (flags & TSFM_ATTN_DEVICE_PTRS) {
        if (!aligned(q, 16) || !aligned(o, 16)) return fail(TSFM_E_UNSUPPORTED, "device q/o must be 16-byte aligned");
        e = tsfm::launch_kv_attend(L, bf16, q, q_tok, q_batch, o, o_tok, o_batch, n_q, q_pos0, n_k, scale,
                                   static_cast<hipStream_t>(stream));
        if (e != hipSuccess) return hip_fail(e, "KV attend launch");
        return TSFM_OK;
    }
    const size_t q_n = span(c->B, n_q, q_tok, q_batch, row) * 2, o_n = span(c->B, n_q, o_tok, o_batch, row) * 2;
    Plan plan;
    const size_t q_at = plan.take(q_n), o_at = plan.take(o_n);
    rc = ensure_buf(ctx, plan.off);
    if (rc != TSFM_OK) return rc;
    char* base = static_cast<char*>(ctx->buf);
    hipStream_t s = ctx->stream;
    if ((e = hipMemcpyAsync(base + q_at, q, q_n, hipMemcpyHostToDevice, s)) != hipSuccess) return hip_fail(e, "host-to-device copy");
    e = tsfm::launch_kv_attend(L, bf16, base + q_at, q_tok, q_batch, base + o_at, o_tok, o_batch, n_q, q_pos0, n_k, scale, s);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "KV attend launch");
    }
    if ((e = copy_rows_d2h(o, base + o_at, c->B, n_q, o_batch * 2, o_tok * 2, row * 2, s)) != hipSuccess)
        return hip_fail(e, "device-to-host copy");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronise");
    return TSFM_OK;
}

int tsfm_kv_append_attend(tsfm_kv_cache* c, const void* k, int64_t k_tok, int64_t k_batch, const void* v,
                          int64_t v_tok, int64_t v_batch, const void* q, int64_t q_tok, int64_t q_batch, void* o,
                          int64_t o_tok, int64_t o_batch, int32_t n_new, float scale, uint32_t flags, void* stream) {
    if (c == nullptr || k == nullptr || v == nullptr || q == nullptr || o == nullptr)
        return fail(TSFM_E_INVALID, "NULL argument");
    if (n_new < 0) return fail(TSFM_E_INVALID, "negative size");
    if (n_new == 0) return TSFM_OK;
    const int32_t pos0 = c->len;
    if (!(flags & TSFM_ATTN_DEVICE_PTRS) || n_new != tsfm::kKvFusedBlock || pos0 % 32 != 0) {
        // Host pointers (staged by each call), or a block other than 32 tokens on a 32-key boundary:
        // the two calls.
        int rc = tsfm_kv_append(c, k, k_tok, k_batch, v, v_tok, v_batch, n_new, flags, stream);
        if (rc != TSFM_OK) return rc;
        return tsfm_kv_attend(c, q, q_tok, q_batch, o, o_tok, o_batch, n_new, pos0, scale, flags, stream);
    }
    // The checks of both calls, then one launch.
    if (k_tok < 0 || k_batch < 0 || v_tok < 0 || v_batch < 0 || q_tok < 0 || q_batch < 0 || o_tok < 0 || o_batch < 0)
        return fail(TSFM_E_INVALID, "negative stride");
    if ((int64_t)pos0 + n_new > c->cap)
        return fail(TSFM_E_INVALID, "append of %d exceeds capacity %d (len %d)", n_new, c->cap, c->len);
    if (k_tok % 8 || k_batch % 8 || v_tok % 8 || v_batch % 8 || q_tok % 8 || q_batch % 8 || o_tok % 8 || o_batch % 8)
        return fail(TSFM_E_UNSUPPORTED, "strides must be multiples of 16 bytes");
    const int64_t row = (int64_t)c->H * c->D;
    if (o_tok < row && n_new > 1) return fail(TSFM_E_INVALID, "o token stride smaller than heads * head_dim");
    if (span_checked(c->B, n_new, k_tok, k_batch, row) < 0 || span_checked(c->B, n_new, v_tok, v_batch, row) < 0 ||
        span_checked(c->B, n_new, q_tok, q_batch, row) < 0 || span_checked(c->B, n_new, o_tok, o_batch, row) < 0)
        return fail(TSFM_E_UNSUPPORTED, "a view spans more than 2^46 elements");
    if (!aligned(k, 16) || !aligned(v, 16) || !aligned(q, 16) || !aligned(o, 16))
        return fail(TSFM_E_UNSUPPORTED, "device k/v/q/o must be 16-byte aligned");
    if (!(scale >= 0.f)) return fail(TSFM_E_UNSUPPORTED, "half-precision attention needs a non-negative scale");
    int rc = ensure_ready();
    if (rc != TSFM_OK) return rc;
    tsfm::KvLayout L{c->k, c->v, c->B, c->H, c->cap};
    const tsfm::KvNew nw{k, k_tok, k_batch, v, v_tok, v_batch};
    const hipError_t e = tsfm::launch_kv_append_attend(L, c->dtype == TSFM_DTYPE_BF16, nw, q, q_tok, q_batch, o, o_tok,
                                                       o_batch, n_new, pos0, scale, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "KV append-attend launch");
    c->len += n_new;
    return TSFM_OK;
}

}  // extern "C"
