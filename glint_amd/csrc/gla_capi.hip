// gla_capi.hip -- C ABI entry points: context, device memory, KV storage
// objects and argument validation. Kernels live in gla_decode.hip,
// gla_prefill.hip and gla_kvstore.hip.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <exception>
#include <mutex>
#include <new>

#include "gla_internal.h"

namespace gla {

static thread_local std::string g_last_error;

int set_error(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

KvLayout layout_of(const gla_kv *kv) {
    KvLayout L;
    const int d = kv->head_dim;
    L.page_stride = kv->page_bytes;
    L.head_stride = kv->head_bytes;
    if (kv->dtype == GLA_KV_F32) {
        L.k = kv->base;
        L.v = kv->base + (size_t)GLA_PAGE_SIZE * d * 4;
        L.ks = nullptr;
        L.vs = nullptr;
        L.row_stride = d * 4;
        L.srow_stride = 0;
    } else {
        L.k = kv->base;
        L.v = kv->base + (size_t)GLA_PAGE_SIZE * d;
        L.ks = kv->base + (size_t)GLA_PAGE_SIZE * d * 2;
        L.vs = L.ks + (size_t)GLA_PAGE_SIZE * (d / 32) * 2;
        L.row_stride = d;
        L.srow_stride = (d / 32) * 2;
    }
    return L;
}

// Grow *ptr to at least `need` bytes (doubling). The old buffer is retired,
// not freed: kernels still queued on the stream and graphs captured from it
// keep their pointers, so growing needs no synchronisation.
static int grow(gla_ctx *ctx, void **ptr, size_t *cur, size_t need, bool pinned) {
    if (need <= *cur) return GLA_OK;
    size_t want = std::max(need, *cur * 2);
    void *fresh = nullptr;
    hipError_t e = pinned ? hipHostMalloc(&fresh, want, hipHostMallocDefault) : hipMalloc(&fresh, want);
    if (e != hipSuccess)
        return set_error(GLA_ERR_BUFFER, "allocation of %zu bytes failed: %s", want, hipGetErrorString(e));
    if (*ptr) ctx->retired.emplace_back(*ptr, pinned);
    *ptr = fresh;
    *cur = want;
    return GLA_OK;
}

int ensure_scratch(gla_ctx *ctx, size_t bytes, void **out) {
    *out = nullptr;
    gla_ctx::StreamScratch *ss = nullptr;
    for (auto &e : ctx->scratch)
        if (e.stream == ctx->stream) ss = &e;
    if (!ss || bytes > ss->bytes) {
        // growing allocates, which a stream capture does not allow: refuse
        // clearly instead of failing inside hipMalloc
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        GLA_CHECK_HIP(hipStreamIsCapturing(ctx->stream, &cs), GLA_ERR_DEVICE);
        if (cs != hipStreamCaptureStatusNone)
            return set_error(GLA_ERR_INVALID,
                             "this call needs %zu bytes of scratch on a stream being captured, which holds %zu: "
                             "scratch must be sized before capture (run the same call once eagerly first)",
                             bytes, ss ? ss->bytes : (size_t)0);
    }
    if (!ss) {
        ctx->scratch.push_back({ctx->stream, nullptr, 0});
        ss = &ctx->scratch.back();
    }
    int rc = grow(ctx, &ss->ptr, &ss->bytes, bytes, false);
    if (rc == GLA_OK) *out = ss->ptr;
    return rc;
}

int decode_arrivals(gla_ctx *ctx, const DecodeLaunch &d, size_t n, int32_t **out) {
    *out = nullptr;
    if (d.scratch) {
        if (n > d.arrivals_cap)
            return set_error(GLA_ERR_INVALID,
                             "decode needs %zu arrival counters (sequences x KV heads x head groups); the fixed "
                             "array holds %zu",
                             n, d.arrivals_cap);
        *out = d.arrivals;
        return GLA_OK;
    }
    return ensure_arrivals(ctx, n, out);
}

int ensure_arrivals(gla_ctx *ctx, size_t n, int32_t **out) {
    *out = nullptr;
    gla_ctx::StreamScratch *ss = nullptr;
    for (auto &e : ctx->scratch)
        if (e.stream == ctx->stream) ss = &e;
    if (ss && n <= ss->n_arrivals) {
        *out = ss->arrivals;
        return GLA_OK;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    GLA_CHECK_HIP(hipStreamIsCapturing(ctx->stream, &cs), GLA_ERR_DEVICE);
    if (cs != hipStreamCaptureStatusNone)
        return set_error(GLA_ERR_INVALID,
                         "this call needs %zu arrival counters on a stream being captured, which holds %zu: they "
                         "must be sized before capture (run the same call once eagerly first)",
                         n, ss ? ss->n_arrivals : (size_t)0);
    if (!ss) {
        ctx->scratch.push_back({ctx->stream, nullptr, 0});
        ss = &ctx->scratch.back();
    }
    const size_t want = std::max<size_t>(n, std::max<size_t>(1024, 2 * ss->n_arrivals));
    void *fresh = nullptr;
    hipError_t e = hipMalloc(&fresh, want * sizeof(int32_t));
    if (e != hipSuccess)
        return set_error(GLA_ERR_BUFFER, "allocation of %zu arrival counters failed: %s", want, hipGetErrorString(e));
    // (queued on the stream: ordered before every launch that uses them)
    e = hipMemsetAsync(fresh, 0, want * sizeof(int32_t), ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(fresh);
        return set_error(GLA_ERR_DEVICE, "zeroing the arrival counters failed: %s", hipGetErrorString(e));
    }
    if (ss->arrivals) ctx->retired.emplace_back(ss->arrivals, false);
    ss->arrivals = (int32_t *)fresh;
    ss->n_arrivals = want;
    *out = ss->arrivals;
    return GLA_OK;
}

int decode_scratch(gla_ctx *ctx, const DecodeLaunch &d, size_t bytes, void **out) {
    if (!d.scratch) return ensure_scratch(ctx, bytes, out);
    *out = nullptr;
    if (bytes > d.scratch_cap)
        return set_error(GLA_ERR_INVALID, "decode needs %zu bytes of scratch; the fixed buffer holds %zu", bytes,
                         d.scratch_cap);
    *out = d.scratch;
    return GLA_OK;
}
int ensure_dstage(gla_ctx *ctx, size_t bytes) {
    return grow(ctx, &ctx->dstage, &ctx->dstage_bytes, bytes, false);
}
int ensure_hstage(gla_ctx *ctx, size_t bytes) {
    return grow(ctx, &ctx->hstage, &ctx->hstage_bytes, bytes, true);
}

static bool head_dim_ok(int d) { return d == 64 || d == 128 || d == 256; }

// Split partials of gla_decode_noalloc: one array per GPU, held until the
// process ends. In host code `scratch` is only a stand-in for the symbol;
// kernels get the device address gla_create resolved for the device.
static __device__ __align__(256) uint8_t scratch[GLA_DECODE_NOALLOC_SCRATCH_BYTES];
// Its arrival counters (zero-initialised when the code object loads; every
// call leaves them at zero). Same stand-in rule as `scratch`.
static __device__ __align__(256) int32_t scratch_arrivals[GLA_DECODE_NOALLOC_UNITS];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];
static void *g_arrivals_ptr[kMaxDevices];
static hipError_t g_scratch_err[kMaxDevices];

// Resolve `scratch` and `scratch_arrivals` on `device` (which must be
// current), once per device.
static void resolve_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return;
    void *ptr = nullptr, *arr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e == hipSuccess) e = hipGetSymbolAddress(&arr, HIP_SYMBOL(scratch_arrivals));
    g_scratch_err[device] = e;
    if (e == hipSuccess) {
        g_scratch_ptr[device] = ptr;
        g_arrivals_ptr[device] = arr;
    }
}

// The device address of `device`'s array, or NULL with the error set.
static void *scratch_of(int device) {
    if (device < 0 || device >= kMaxDevices) {
        set_error(GLA_ERR_DEVICE, "gla_decode_noalloc: device %d beyond the %d the library tracks", device,
                  kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device])
        set_error(GLA_ERR_DEVICE, "gla_decode_noalloc: the static scratch of device %d has no address (%s)", device,
                  hipGetErrorString(g_scratch_err[device]));
    return g_scratch_ptr[device];
}
static int32_t *arrivals_of(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return (device >= 0 && device < kMaxDevices) ? (int32_t *)g_arrivals_ptr[device] : nullptr;
}

// Waits for the context's stream when it goes out of scope unless released:
// a host-pointer entry point that queued a copy out of the pinned staging
// buffer and then fails must not return while that copy is pending (the
// next call rewrites the staging buffer).
struct SyncOnExit {
    hipStream_t stream;
    bool armed = true;
    explicit SyncOnExit(hipStream_t s) : stream(s) {}
    ~SyncOnExit() {
        if (armed) (void)hipStreamSynchronize(stream);
    }
};

static size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace gla

using namespace gla;

#define GLA_GUARD_BEGIN try {
#define GLA_GUARD_END                                                         \
    }                                                                         \
    catch (const std::bad_alloc &) {                                          \
        return set_error(GLA_ERR_BUFFER, "host allocation failed");           \
    }                                                                         \
    catch (const std::exception &ex) {                                        \
        return set_error(GLA_ERR_DEVICE, "internal error: %s", ex.what());    \
    }                                                                         \
    catch (...) {                                                             \
        return set_error(GLA_ERR_DEVICE, "internal error at the C boundary"); \
    }

#define GLA_REQUIRE(cond, ...)                                        \
    do {                                                              \
        if (!(cond)) return set_error(GLA_ERR_INVALID, __VA_ARGS__); \
    } while (0)

extern "C" {

const char *gla_last_error(void) { return g_last_error.c_str(); }

int gla_create(int device, gla_ctx **out) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(out != nullptr, "gla_create: out is NULL");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return set_error(GLA_ERR_NO_DEVICE, "no HIP device found (%s)",
                         e == hipSuccess ? "device count 0" : hipGetErrorString(e));
    GLA_REQUIRE(device >= 0 && device < n, "gla_create: device %d out of range (have %d)", device, n);
    GLA_CHECK_HIP(hipSetDevice(device), GLA_ERR_DEVICE);
    resolve_scratch(device);  // the static scratch of gla_decode_noalloc
    gla_ctx *ctx = new gla_ctx();
    ctx->device = device;
    if (hipDeviceGetAttribute(&ctx->n_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        ctx->n_cu = 256;
    e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return set_error(GLA_ERR_DEVICE, "hipStreamCreate: %s", hipGetErrorString(e));
    }
    ctx->stream = ctx->own_stream;
    *out = ctx;
    clear_error();
    return GLA_OK;
    GLA_GUARD_END
}

int gla_destroy(gla_ctx *ctx) {
    GLA_GUARD_BEGIN
    if (!ctx) return GLA_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (const auto &e : ctx->scratch) {
        if (e.ptr) (void)hipFree(e.ptr);
        if (e.arrivals) (void)hipFree(e.arrivals);
    }
    for (gla_kv *kv : ctx->kvs) {
        if (kv->base) (void)hipFree(kv->base);
        kv->base = nullptr;
        kv->ctx = nullptr;
    }
    for (gla_q8w *w : ctx->q8ws) detach_q8w(w);
    if (ctx->dstage) (void)hipFree(ctx->dstage);
    if (ctx->hstage) (void)hipHostFree(ctx->hstage);
    for (const auto &r : ctx->retired) {
        if (r.second)
            (void)hipHostFree(r.first);
        else
            (void)hipFree(r.first);
    }
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return GLA_OK;
    GLA_GUARD_END
}

int gla_set_stream(gla_ctx *ctx, void *hip_stream) {
    GLA_REQUIRE(ctx, "gla_set_stream: ctx is NULL");
    ctx->stream = hip_stream ? (hipStream_t)hip_stream : ctx->own_stream;
    return GLA_OK;
}

void *gla_get_stream(gla_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int gla_release_stream(gla_ctx *ctx, void *hip_stream) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx, "gla_release_stream: ctx is NULL");
    const hipStream_t st = hip_stream ? (hipStream_t)hip_stream : ctx->own_stream;
    auto it = std::find_if(ctx->scratch.begin(), ctx->scratch.end(),
                           [&](const gla_ctx::StreamScratch &e) { return e.stream == st; });
    if (ctx->stream == st && st != ctx->own_stream) ctx->stream = ctx->own_stream;
    if (it == ctx->scratch.end()) return GLA_OK;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    GLA_CHECK_HIP(hipStreamSynchronize(st), GLA_ERR_KERNEL);
    if (it->ptr) (void)hipFree(it->ptr);
    if (it->arrivals) (void)hipFree(it->arrivals);
    ctx->scratch.erase(it);
    return GLA_OK;
    GLA_GUARD_END
}

int gla_sync(gla_ctx *ctx) {
    GLA_REQUIRE(ctx, "gla_sync: ctx is NULL");
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_KERNEL);
    return GLA_OK;
}

int gla_device_cu_count(gla_ctx *ctx) { return ctx ? ctx->n_cu : 0; }

int gla_dev_alloc(gla_ctx *ctx, size_t bytes, void **out) {
    GLA_REQUIRE(ctx && out, "gla_dev_alloc: NULL argument");
    *out = nullptr;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    GLA_CHECK_HIP(hipMalloc(out, bytes ? bytes : 16), GLA_ERR_BUFFER);
    return GLA_OK;
}

int gla_dev_free(gla_ctx *ctx, void *ptr) {
    GLA_REQUIRE(ctx, "gla_dev_free: ctx is NULL");
    if (!ptr) return GLA_OK;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_KERNEL);
    GLA_CHECK_HIP(hipFree(ptr), GLA_ERR_BUFFER);
    return GLA_OK;
}

int gla_memcpy_htod(gla_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes) {
    GLA_REQUIRE(ctx && (bytes == 0 || (dst_dev && src_host)), "gla_memcpy_htod: NULL argument");
    if (bytes == 0) return GLA_OK;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    GLA_CHECK_HIP(hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream), GLA_ERR_BUFFER);
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_BUFFER);
    return GLA_OK;
}

int gla_memcpy_dtoh(gla_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes) {
    GLA_REQUIRE(ctx && (bytes == 0 || (dst_host && src_dev)), "gla_memcpy_dtoh: NULL argument");
    if (bytes == 0) return GLA_OK;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    GLA_CHECK_HIP(hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream), GLA_ERR_BUFFER);
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_BUFFER);
    return GLA_OK;
}

// A storage or weight handle used with `ctx` must have been created on it (and
// not be detached by the context's destruction).
static int check_owner(const gla_ctx *ctx, const gla_kv *kv, const char *fn) {
    if (kv->ctx != ctx)
        return set_error(GLA_ERR_INVALID, "%s: the KV storage belongs to %s", fn,
                         kv->ctx ? "another context" : "a destroyed context");
    return GLA_OK;
}

static int kv_alloc(gla_ctx *ctx, gla_kv *kv) {
    const int d = kv->head_dim;
    kv->kv_dim = kv->n_kv_heads * d;
    kv->head_bytes = kv->dtype == GLA_KV_F32 ? (int64_t)GLA_PAGE_SIZE * d * 4 * 2 : (int64_t)34 * d;
    kv->page_bytes = kv->head_bytes * kv->n_kv_heads;
    size_t bytes = (size_t)kv->page_bytes * (size_t)kv->n_pages;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 256);
    if (e != hipSuccess)
        return set_error(GLA_ERR_BUFFER, "KV storage of %zu bytes: %s", bytes, hipGetErrorString(e));
    kv->base = (uint8_t *)p;
    kv->ctx = ctx;
    if (bytes) {
        int rc = launch_zero_pages(ctx, kv, 0, kv->n_pages);
        if (rc != GLA_OK) {
            (void)hipFree(p);
            return rc;
        }
        e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return set_error(GLA_ERR_KERNEL, "zeroing KV storage: %s", hipGetErrorString(e));
        }
    }
    return GLA_OK;
}

int gla_kv_cache_create(gla_ctx *ctx, gla_kv_dtype dtype, int n_seqs, int n_layers, int max_seq_len,
                        int n_kv_heads, int head_dim, gla_kv **out) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && out, "gla_kv_cache_create: NULL argument");
    *out = nullptr;
    GLA_REQUIRE(dtype == GLA_KV_F32 || dtype == GLA_KV_Q8_0, "gla_kv_cache_create: bad dtype %d", (int)dtype);
    GLA_REQUIRE(head_dim_ok(head_dim), "unsupported head_dim %d (supported: 64, 128, 256)", head_dim);
    GLA_REQUIRE(n_seqs > 0 && n_layers > 0 && max_seq_len > 0 && n_kv_heads > 0,
                "gla_kv_cache_create: sizes must be positive");
    gla_kv *kv = new gla_kv();
    kv->is_pool = false;
    kv->dtype = dtype;
    kv->n_kv_heads = n_kv_heads;
    kv->head_dim = head_dim;
    kv->n_seqs = n_seqs;
    kv->n_layers = n_layers;
    kv->max_seq = max_seq_len;
    kv->pages_per_layer = (max_seq_len + GLA_PAGE_SIZE - 1) / GLA_PAGE_SIZE;
    kv->n_pages = (int64_t)n_seqs * n_layers * kv->pages_per_layer;
    int rc = kv_alloc(ctx, kv);
    if (rc != GLA_OK) {
        delete kv;
        return rc;
    }
    ctx->kvs.push_back(kv);
    *out = kv;
    return GLA_OK;
    GLA_GUARD_END
}

int gla_pool_create(gla_ctx *ctx, gla_kv_dtype dtype, int n_kv_heads, int head_dim, int capacity_pages,
                    gla_kv **out) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && out, "gla_pool_create: NULL argument");
    *out = nullptr;
    GLA_REQUIRE(dtype == GLA_KV_F32 || dtype == GLA_KV_Q8_0, "gla_pool_create: bad dtype %d", (int)dtype);
    GLA_REQUIRE(head_dim_ok(head_dim), "unsupported head_dim %d (supported: 64, 128, 256)", head_dim);
    GLA_REQUIRE(n_kv_heads > 0 && capacity_pages > 0, "gla_pool_create: sizes must be positive");
    gla_kv *kv = new gla_kv();
    kv->is_pool = true;
    kv->dtype = dtype;
    kv->n_kv_heads = n_kv_heads;
    kv->head_dim = head_dim;
    kv->n_pages = capacity_pages;
    int rc = kv_alloc(ctx, kv);
    if (rc != GLA_OK) {
        delete kv;
        return rc;
    }
    ctx->kvs.push_back(kv);
    *out = kv;
    return GLA_OK;
    GLA_GUARD_END
}

int gla_kv_destroy(gla_kv *kv) {
    GLA_GUARD_BEGIN
    if (!kv) return GLA_OK;
    if (gla_ctx *ctx = kv->ctx) {  // else its context already freed the storage
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        if (kv->base) (void)hipFree(kv->base);
        ctx->kvs.erase(std::remove(ctx->kvs.begin(), ctx->kvs.end(), kv), ctx->kvs.end());
    }
    delete kv;
    return GLA_OK;
    GLA_GUARD_END
}

int64_t gla_kv_row_id(const gla_kv *kv, int seq, int layer, int pos) {
    if (!kv || kv->is_pool) return -1;
    if (seq < 0 || seq >= kv->n_seqs || layer < 0 || layer >= kv->n_layers || pos < 0 || pos >= kv->max_seq)
        return -1;
    int64_t page = ((int64_t)seq * kv->n_layers + layer) * kv->pages_per_layer + pos / GLA_PAGE_SIZE;
    return page * GLA_PAGE_SIZE + pos % GLA_PAGE_SIZE;
}

int64_t gla_kv_row_bytes(const gla_kv *kv) {
    if (!kv) return -1;
    return kv->dtype == GLA_KV_F32 ? (int64_t)kv->kv_dim * 4 : (int64_t)((kv->kv_dim + 31) / 32) * 34;
}

static int check_rows_host(const gla_kv *kv, const int64_t *rows, int n) {
    const int64_t limit = kv->n_pages * GLA_PAGE_SIZE;
    for (int i = 0; i < n; i++)
        if (rows[i] < 0 || rows[i] >= limit)
            return set_error(GLA_ERR_INVALID, "row id %lld out of range [0, %lld)", (long long)rows[i],
                             (long long)limit);
    return GLA_OK;
}

int gla_kv_write_rows(gla_ctx *ctx, gla_kv *kv, const int64_t *rows_dev, const float *k_dev,
                      const float *v_dev, int n_rows) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && kv && n_rows >= 0, "gla_kv_write_rows: bad argument");
    if (int rc = check_owner(ctx, kv, "gla_kv_write_rows")) return rc;
    if (n_rows == 0) return GLA_OK;
    GLA_REQUIRE(rows_dev && k_dev && v_dev, "gla_kv_write_rows: NULL buffer");
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    return launch_write_rows(ctx, kv, rows_dev, k_dev, v_dev, n_rows);
    GLA_GUARD_END
}

int gla_kv_write_rows_host(gla_ctx *ctx, gla_kv *kv, const int64_t *rows, const float *k, const float *v,
                           int n_rows) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && kv && n_rows >= 0, "gla_kv_write_rows_host: bad argument");
    if (int rc = check_owner(ctx, kv, "gla_kv_write_rows_host")) return rc;
    if (n_rows == 0) return GLA_OK;
    GLA_REQUIRE(rows && k && v, "gla_kv_write_rows_host: NULL buffer");
    int rc = check_rows_host(kv, rows, n_rows);
    if (rc != GLA_OK) return rc;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    const size_t rb = align_up((size_t)n_rows * 8, 256);
    const size_t fb = align_up((size_t)n_rows * kv->kv_dim * 4, 256);
    const size_t total = rb + 2 * fb;
    if ((rc = ensure_dstage(ctx, total)) != GLA_OK) return rc;
    if ((rc = ensure_hstage(ctx, total)) != GLA_OK) return rc;
    uint8_t *h = (uint8_t *)ctx->hstage;
    uint8_t *d = (uint8_t *)ctx->dstage;
    memcpy(h, rows, (size_t)n_rows * 8);
    memcpy(h + rb, k, (size_t)n_rows * kv->kv_dim * 4);
    memcpy(h + rb + fb, v, (size_t)n_rows * kv->kv_dim * 4);
    SyncOnExit pending(ctx->stream);
    GLA_CHECK_HIP(hipMemcpyAsync(d, h, total, hipMemcpyHostToDevice, ctx->stream), GLA_ERR_BUFFER);
    rc = launch_write_rows(ctx, kv, (const int64_t *)d, (const float *)(d + rb), (const float *)(d + rb + fb),
                           n_rows);
    if (rc != GLA_OK) return rc;
    pending.armed = false;
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_KERNEL);
    return GLA_OK;
    GLA_GUARD_END
}

int gla_kv_export_rows_host(gla_ctx *ctx, const gla_kv *kv, const int64_t *rows, int n_rows, uint8_t *k_out,
                            uint8_t *v_out) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && kv && n_rows >= 0, "gla_kv_export_rows_host: bad argument");
    if (int rc = check_owner(ctx, kv, "gla_kv_export_rows_host")) return rc;
    if (n_rows == 0) return GLA_OK;
    GLA_REQUIRE(rows && k_out && v_out, "gla_kv_export_rows_host: NULL buffer");
    int rc = check_rows_host(kv, rows, n_rows);
    if (rc != GLA_OK) return rc;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    const size_t row_bytes = (size_t)gla_kv_row_bytes(kv);
    const size_t rb = align_up((size_t)n_rows * 8, 256);
    const size_t ob = align_up((size_t)n_rows * row_bytes, 256);
    const size_t total = rb + 2 * ob;
    if ((rc = ensure_dstage(ctx, total)) != GLA_OK) return rc;
    if ((rc = ensure_hstage(ctx, total)) != GLA_OK) return rc;
    uint8_t *h = (uint8_t *)ctx->hstage;
    uint8_t *d = (uint8_t *)ctx->dstage;
    memcpy(h, rows, (size_t)n_rows * 8);
    SyncOnExit pending(ctx->stream);
    GLA_CHECK_HIP(hipMemcpyAsync(d, h, (size_t)n_rows * 8, hipMemcpyHostToDevice, ctx->stream), GLA_ERR_BUFFER);
    rc = launch_export_rows(ctx, kv, (const int64_t *)d, n_rows, d + rb, d + rb + ob);
    if (rc != GLA_OK) return rc;
    GLA_CHECK_HIP(hipMemcpyAsync(h + rb, d + rb, 2 * ob, hipMemcpyDeviceToHost, ctx->stream), GLA_ERR_BUFFER);
    pending.armed = false;
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_KERNEL);
    memcpy(k_out, h + rb, (size_t)n_rows * row_bytes);
    memcpy(v_out, h + rb + ob, (size_t)n_rows * row_bytes);
    return GLA_OK;
    GLA_GUARD_END
}

int gla_kv_import_rows_host(gla_ctx *ctx, gla_kv *kv, const int64_t *rows, int n_rows, const uint8_t *k_in,
                            const uint8_t *v_in) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && kv && n_rows >= 0, "gla_kv_import_rows_host: bad argument");
    if (int rc = check_owner(ctx, kv, "gla_kv_import_rows_host")) return rc;
    if (n_rows == 0) return GLA_OK;
    GLA_REQUIRE(rows && k_in && v_in, "gla_kv_import_rows_host: NULL buffer");
    int rc = check_rows_host(kv, rows, n_rows);
    if (rc != GLA_OK) return rc;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    const size_t row_bytes = (size_t)gla_kv_row_bytes(kv);
    const size_t rb = align_up((size_t)n_rows * 8, 256);
    const size_t ib = align_up((size_t)n_rows * row_bytes, 256);
    const size_t total = rb + 2 * ib;
    if ((rc = ensure_dstage(ctx, total)) != GLA_OK) return rc;
    if ((rc = ensure_hstage(ctx, total)) != GLA_OK) return rc;
    uint8_t *h = (uint8_t *)ctx->hstage;
    uint8_t *d = (uint8_t *)ctx->dstage;
    memcpy(h, rows, (size_t)n_rows * 8);
    memcpy(h + rb, k_in, (size_t)n_rows * row_bytes);
    memcpy(h + rb + ib, v_in, (size_t)n_rows * row_bytes);
    SyncOnExit pending(ctx->stream);
    GLA_CHECK_HIP(hipMemcpyAsync(d, h, total, hipMemcpyHostToDevice, ctx->stream), GLA_ERR_BUFFER);
    rc = launch_import_rows(ctx, kv, (const int64_t *)d, n_rows, d + rb, d + rb + ib);
    if (rc != GLA_OK) return rc;
    pending.armed = false;
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_KERNEL);
    return GLA_OK;
    GLA_GUARD_END
}

int gla_pool_copy_page(gla_ctx *ctx, gla_kv *pool, int src_page, int dst_page) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && pool && pool->is_pool, "gla_pool_copy_page: needs a pool");
    if (int rc = check_owner(ctx, pool, "gla_pool_copy_page")) return rc;
    GLA_REQUIRE(src_page >= 0 && src_page < pool->n_pages && dst_page >= 0 && dst_page < pool->n_pages,
                "gla_pool_copy_page: page out of range");
    if (src_page == dst_page) return GLA_OK;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    return launch_copy_page(ctx, pool, src_page, dst_page);
    GLA_GUARD_END
}

int gla_pool_zero_page(gla_ctx *ctx, gla_kv *pool, int page) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && pool && pool->is_pool, "gla_pool_zero_page: needs a pool");
    if (int rc = check_owner(ctx, pool, "gla_pool_zero_page")) return rc;
    GLA_REQUIRE(page >= 0 && page < pool->n_pages, "gla_pool_zero_page: page out of range");
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    return launch_zero_pages(ctx, pool, page, 1);
    GLA_GUARD_END
}

long gla_window_start(long pos, long sliding_window, int alternating, int layer) {
    if (alternating && (layer % 2) != 0) return 0;
    if (sliding_window <= 0) return 0;
    long w = pos - sliding_window + 1;
    return w > 0 ? w : 0;
}

static int page_map_of(const gla_kv *kv, int layer, const int32_t *seq_slot, const int32_t *page_table,
                       int pt_stride, PageMap *pm) {
    memset(pm, 0, sizeof(*pm));
    if (kv->is_pool) {
        GLA_REQUIRE(page_table != nullptr, "a pool needs a page table");
        GLA_REQUIRE(pt_stride > 0, "page_table_stride must be positive");
        pm->page_table = page_table;
        pm->pt_stride = pt_stride;
        pm->n_pages = kv->n_pages;
        pm->pos_limit = pt_stride * GLA_PAGE_SIZE;
        pm->n_slots = 1;
    } else {
        GLA_REQUIRE(page_table == nullptr, "contiguous caches take no page table");
        GLA_REQUIRE(layer >= 0 && layer < kv->n_layers, "layer %d out of range [0, %d)", layer, kv->n_layers);
        pm->seq_slot = seq_slot;
        pm->seq_page_stride = (int64_t)kv->n_layers * kv->pages_per_layer;
        pm->layer_page_off = (int64_t)layer * kv->pages_per_layer;
        pm->n_pages = kv->n_pages;
        pm->pos_limit = kv->max_seq;
        pm->n_slots = kv->n_seqs;
    }
    return GLA_OK;
}

// Validate gla_decode_args and fill the launch; *nothing = true when the
// batch is empty (GLA_OK, nothing to launch).
static int decode_launch_of(gla_ctx *ctx, const gla_decode_args *a, const char *fn, DecodeLaunch *d,
                            bool *nothing) {
    *nothing = false;
    GLA_REQUIRE(ctx && a && a->kv, "%s: NULL argument", fn);
    const gla_kv *kv = a->kv;
    if (int rc = check_owner(ctx, kv, fn)) return rc;
    GLA_REQUIRE(a->n_seqs >= 0, "%s: n_seqs < 0", fn);
    if (a->n_seqs == 0) {
        *nothing = true;
        return GLA_OK;
    }
    GLA_REQUIRE(a->q && a->out && a->kv_start && a->kv_len, "%s: NULL buffer", fn);
    GLA_REQUIRE(a->n_heads > 0 && a->n_heads % kv->n_kv_heads == 0,
                "%s: n_heads %d is not a multiple of n_kv_heads %d", fn, a->n_heads, kv->n_kv_heads);
    GLA_REQUIRE(a->max_kv_len >= 0, "%s: max_kv_len < 0", fn);
    GLA_REQUIRE(!kv->is_pool || a->page_table_stride * GLA_PAGE_SIZE >= a->max_kv_len,
                "%s: page_table_stride %d cannot cover max_kv_len %d", fn, a->page_table_stride, a->max_kv_len);
    GLA_REQUIRE(kv->is_pool || a->max_kv_len <= kv->max_seq, "%s: max_kv_len %d > cache max_seq %d", fn,
                a->max_kv_len, kv->max_seq);
    int rc = page_map_of(kv, a->layer, a->seq_slot, a->page_table, a->page_table_stride, &d->pm);
    if (rc != GLA_OK) return rc;
    d->kv = layout_of(kv);
    d->q8 = kv->dtype == GLA_KV_Q8_0;
    d->head_dim = kv->head_dim;
    d->n_kv_heads = kv->n_kv_heads;
    d->n_seqs = a->n_seqs;
    d->kv_start = a->kv_start;
    d->kv_len = a->kv_len;
    d->max_kv_len = a->max_kv_len;
    d->n_heads = a->n_heads;
    d->scale = a->scale;
    d->softcap = a->softcap;
    d->q = a->q;
    d->out = a->out;
    GLA_REQUIRE((a->kv_start_host == nullptr) == (a->kv_len_host == nullptr),
                "%s: pass both kv_start_host and kv_len_host, or neither", fn);
    d->kv_start_host = a->kv_start_host;
    d->kv_len_host = a->kv_len_host;
    if (a->kv_len_host) {
        // The reference panics on a window outside the storage
        // (src/cache/paged.rs:453-465, src/cache/mod.rs:167-171); with the
        // host copies this is seen before anything is launched.
        const int64_t limit = d->pm.pos_limit;
        for (int b = 0; b < a->n_seqs; b++) {
            const int64_t st = a->kv_start_host[b], len = a->kv_len_host[b];
            GLA_REQUIRE(st >= 0 && len >= 0 && len <= a->max_kv_len && st + len <= limit,
                        "%s: sequence %d attends positions [%lld, %lld), outside [0, %lld) or longer than "
                        "max_kv_len %d",
                        fn, b, (long long)st, (long long)(st + len), (long long)limit, a->max_kv_len);
        }
    }
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    if (a->kv_len_host) {
        // The host lengths size the launch; a captured graph would replay
        // that sizing after the device lengths have grown.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        GLA_CHECK_HIP(hipStreamIsCapturing(ctx->stream, &cs), GLA_ERR_DEVICE);
        GLA_REQUIRE(cs == hipStreamCaptureStatusNone,
                    "%s: host lengths are not allowed while the stream is being captured (a graph replay would "
                    "keep the launch sized for them); pass max_kv_len = the capacity and no host lengths",
                    fn);
    }
    return GLA_OK;
}

int gla_decode(gla_ctx *ctx, const gla_decode_args *a) {
    GLA_GUARD_BEGIN
    DecodeLaunch d;
    bool nothing = false;
    int rc = decode_launch_of(ctx, a, "gla_decode", &d, &nothing);
    if (rc != GLA_OK || nothing) return rc;
    return launch_decode(ctx, d);
    GLA_GUARD_END
}

int gla_decode_noalloc(gla_ctx *ctx, const gla_decode_args *a) {
    GLA_GUARD_BEGIN
    DecodeLaunch d;
    bool nothing = false;
    int rc = decode_launch_of(ctx, a, "gla_decode_noalloc", &d, &nothing);
    if (rc != GLA_OK || nothing) return rc;
    d.scratch = scratch_of(ctx->device);
    if (!d.scratch) return GLA_ERR_DEVICE;
    d.scratch_cap = GLA_DECODE_NOALLOC_SCRATCH_BYTES;
    d.arrivals = arrivals_of(ctx->device);
    d.arrivals_cap = GLA_DECODE_NOALLOC_UNITS;
    return launch_decode(ctx, d);
    GLA_GUARD_END
}

int gla_prefill(gla_ctx *ctx, const gla_prefill_args *a) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && a && a->kv, "gla_prefill: NULL argument");
    const gla_kv *kv = a->kv;
    if (int rc = check_owner(ctx, kv, "gla_prefill")) return rc;
    GLA_REQUIRE(a->n_seqs >= 0, "gla_prefill: n_seqs < 0");
    if (a->n_seqs == 0 || a->max_q_len == 0) return GLA_OK;
    GLA_REQUIRE(a->q && a->out && a->q_start && a->pos_offset, "gla_prefill: NULL buffer");
    GLA_REQUIRE(a->max_q_len > 0, "gla_prefill: max_q_len < 0");
    GLA_REQUIRE(a->n_heads > 0 && a->n_heads % kv->n_kv_heads == 0,
                "gla_prefill: n_heads %d is not a multiple of n_kv_heads %d", a->n_heads, kv->n_kv_heads);
    GLA_REQUIRE(a->precision == GLA_PREC_F32 || a->precision == GLA_PREC_BF16, "gla_prefill: bad precision");
    PrefillLaunch p;
    int rc = page_map_of(kv, a->layer, a->seq_slot, a->page_table, a->page_table_stride, &p.pm);
    if (rc != GLA_OK) return rc;
    p.kv = layout_of(kv);
    p.q8 = kv->dtype == GLA_KV_Q8_0;
    p.head_dim = kv->head_dim;
    p.n_kv_heads = kv->n_kv_heads;
    p.n_seqs = a->n_seqs;
    p.q_start = a->q_start;
    p.pos_offset = a->pos_offset;
    p.max_q_len = a->max_q_len;
    p.n_heads = a->n_heads;
    p.scale = a->scale;
    p.softcap = a->softcap;
    p.sliding_window = a->sliding_window;
    p.precision = a->precision;
    p.q = a->q;
    p.out = a->out;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    return launch_prefill(ctx, p);
    GLA_GUARD_END
}

int gla_attention(gla_ctx *ctx, const float *q, const float *k, const float *v, int n_heads, int n_kv_heads,
                  int head_dim, int seq_len, float scale, float softcap, float *out) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && q && out, "gla_attention: NULL argument");
    GLA_REQUIRE(head_dim_ok(head_dim), "unsupported head_dim %d (supported: 64, 128, 256)", head_dim);
    GLA_REQUIRE(n_kv_heads > 0 && n_heads > 0 && n_heads % n_kv_heads == 0,
                "gla_attention: n_heads %d is not a multiple of n_kv_heads %d", n_heads, n_kv_heads);
    GLA_REQUIRE(seq_len >= 0, "gla_attention: seq_len < 0");
    GLA_REQUIRE(seq_len == 0 || (k && v), "gla_attention: NULL K/V");
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    const size_t kv_dim = (size_t)n_kv_heads * head_dim;
    const size_t qb = align_up((size_t)n_heads * head_dim * 4, 256);
    const size_t pad_rows = (size_t)((seq_len + GLA_PAGE_SIZE - 1) / GLA_PAGE_SIZE) * GLA_PAGE_SIZE;
    const size_t kb = align_up(pad_rows * kv_dim * 4, 256);
    const size_t ib = 256;  // kv_start, kv_len
    const size_t total = 2 * qb + 2 * kb + ib;
    int rc;
    if ((rc = ensure_dstage(ctx, total)) != GLA_OK) return rc;
    if ((rc = ensure_hstage(ctx, total)) != GLA_OK) return rc;
    uint8_t *h = (uint8_t *)ctx->hstage;
    uint8_t *d = (uint8_t *)ctx->dstage;
    // layout of the staging: [q][out][k][v][ints]
    memcpy(h, q, (size_t)n_heads * head_dim * 4);
    if (seq_len) {
        memcpy(h + 2 * qb, k, (size_t)seq_len * kv_dim * 4);
        memcpy(h + 2 * qb + kb, v, (size_t)seq_len * kv_dim * 4);
    }
    int32_t *ints = (int32_t *)(h + 2 * qb + 2 * kb);
    ints[0] = 0;
    ints[1] = seq_len;
    SyncOnExit pending(ctx->stream);
    GLA_CHECK_HIP(hipMemcpyAsync(d, h, qb, hipMemcpyHostToDevice, ctx->stream), GLA_ERR_BUFFER);
    GLA_CHECK_HIP(hipMemcpyAsync(d + 2 * qb, h + 2 * qb, 2 * kb + ib, hipMemcpyHostToDevice, ctx->stream),
                  GLA_ERR_BUFFER);
    // The host K/V keep Glint's flat [pos][kv_head][d] layout: page p is rows
    // 16p .. 16p+15, heads are d floats apart, rows kv_dim floats apart.
    DecodeLaunch dl;
    dl.kv.k = d + 2 * qb;
    dl.kv.v = d + 2 * qb + kb;
    dl.kv.ks = nullptr;
    dl.kv.vs = nullptr;
    dl.kv.page_stride = (int64_t)GLA_PAGE_SIZE * kv_dim * 4;
    dl.kv.head_stride = (int64_t)head_dim * 4;
    dl.kv.row_stride = (int32_t)(kv_dim * 4);
    dl.kv.srow_stride = 0;
    dl.q8 = false;
    dl.head_dim = head_dim;
    dl.n_kv_heads = n_kv_heads;
    memset(&dl.pm, 0, sizeof(dl.pm));
    dl.pm.n_pages = (int64_t)(pad_rows / GLA_PAGE_SIZE);
    dl.pm.pos_limit = seq_len;
    dl.pm.n_slots = 1;
    dl.n_seqs = 1;
    dl.kv_start = (const int32_t *)(d + 2 * qb + 2 * kb);
    dl.kv_len = dl.kv_start + 1;
    dl.max_kv_len = seq_len;
    dl.n_heads = n_heads;
    dl.scale = scale;
    dl.softcap = softcap;
    dl.q = (const float *)d;
    dl.out = (float *)(d + qb);
    rc = launch_decode(ctx, dl);
    if (rc != GLA_OK) return rc;
    GLA_CHECK_HIP(hipMemcpyAsync(h + qb, d + qb, (size_t)n_heads * head_dim * 4, hipMemcpyDeviceToHost,
                                 ctx->stream),
                  GLA_ERR_BUFFER);
    pending.armed = false;
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_KERNEL);
    memcpy(out, h + qb, (size_t)n_heads * head_dim * 4);
    return GLA_OK;
    GLA_GUARD_END
}

int gla_attention_resident(gla_ctx *ctx, const float *q, const gla_kv *cache, int seq, int layer,
                           int window_start, int attend_len, int n_heads, float scale, float softcap,
                           float *out) {
    GLA_GUARD_BEGIN
    GLA_REQUIRE(ctx && q && out && cache, "gla_attention_resident: NULL argument");
    if (int rc = check_owner(ctx, cache, "gla_attention_resident")) return rc;
    GLA_REQUIRE(!cache->is_pool, "gla_attention_resident: needs a contiguous cache");
    GLA_REQUIRE(seq >= 0 && seq < cache->n_seqs, "gla_attention_resident: seq out of range");
    GLA_REQUIRE(window_start >= 0 && attend_len >= 0 && (int64_t)window_start + attend_len <= cache->max_seq,
                "gla_attention_resident: window [%d, %d) outside the cache", window_start,
                window_start + attend_len);
    GLA_REQUIRE(n_heads > 0 && n_heads % cache->n_kv_heads == 0, "gla_attention_resident: bad n_heads");
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    const size_t qb = align_up((size_t)n_heads * cache->head_dim * 4, 256);
    const size_t total = 2 * qb + 256;
    int rc;
    if ((rc = ensure_dstage(ctx, total)) != GLA_OK) return rc;
    if ((rc = ensure_hstage(ctx, total)) != GLA_OK) return rc;
    uint8_t *h = (uint8_t *)ctx->hstage;
    uint8_t *d = (uint8_t *)ctx->dstage;
    memcpy(h, q, (size_t)n_heads * cache->head_dim * 4);
    int32_t *ints = (int32_t *)(h + 2 * qb);
    ints[0] = window_start;
    ints[1] = attend_len;
    ints[2] = seq;
    SyncOnExit pending(ctx->stream);
    GLA_CHECK_HIP(hipMemcpyAsync(d, h, qb, hipMemcpyHostToDevice, ctx->stream), GLA_ERR_BUFFER);
    GLA_CHECK_HIP(hipMemcpyAsync(d + 2 * qb, h + 2 * qb, 256, hipMemcpyHostToDevice, ctx->stream),
                  GLA_ERR_BUFFER);
    DecodeLaunch dl;
    rc = page_map_of(cache, layer, (const int32_t *)(d + 2 * qb) + 2, nullptr, 0, &dl.pm);
    if (rc != GLA_OK) return rc;
    dl.kv = layout_of(cache);
    dl.q8 = cache->dtype == GLA_KV_Q8_0;
    dl.head_dim = cache->head_dim;
    dl.n_kv_heads = cache->n_kv_heads;
    dl.n_seqs = 1;
    dl.kv_start = (const int32_t *)(d + 2 * qb);
    dl.kv_len = dl.kv_start + 1;
    dl.max_kv_len = attend_len;
    dl.n_heads = n_heads;
    dl.scale = scale;
    dl.softcap = softcap;
    dl.q = (const float *)d;
    dl.out = (float *)(d + qb);
    rc = launch_decode(ctx, dl);
    if (rc != GLA_OK) return rc;
    GLA_CHECK_HIP(hipMemcpyAsync(h + qb, d + qb, (size_t)n_heads * cache->head_dim * 4, hipMemcpyDeviceToHost,
                                 ctx->stream),
                  GLA_ERR_BUFFER);
    pending.armed = false;
    GLA_CHECK_HIP(hipStreamSynchronize(ctx->stream), GLA_ERR_KERNEL);
    memcpy(out, h + qb, (size_t)n_heads * cache->head_dim * 4);
    return GLA_OK;
    GLA_GUARD_END
}

}  // extern "C"
