// glint.cpp -- the C++ host layer declared in glint.hpp, over include/glint_attn.h.
#include "glint.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <numeric>

namespace glint {

namespace {

std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

Status check(int rc, const char *what) {
    if (rc == GLA_OK) return {};
    return GlintError::from_status(rc, what);
}

size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

}  // namespace

// ---- GlintError ----------------------------------------------------------------

GlintError GlintError::gpu_adapter_not_found() { return GlintError(Kind::GpuAdapterNotFound, ""); }
GlintError GlintError::gpu_device_error(std::string m) { return GlintError(Kind::GpuDeviceError, std::move(m)); }
GlintError GlintError::gpu_buffer_error(std::string m) { return GlintError(Kind::GpuBufferError, std::move(m)); }
GlintError GlintError::gpu_shader_error(std::string m) { return GlintError(Kind::GpuShaderError, std::move(m)); }
GlintError GlintError::snapshot_cache_size_mismatch(size_t layer, size_t expected, size_t found) {
    return GlintError(Kind::SnapshotCacheSizeMismatch, "", layer, expected, found);
}
GlintError GlintError::kv_page_pool_exhausted(size_t needed, size_t available, size_t capacity) {
    return GlintError(Kind::KvPagePoolExhausted, "", needed, available, capacity);
}

GlintError GlintError::from_status(int status, const char *what) {
    std::string m = std::string(what) + ": " + gla_last_error();
    switch (status) {
    case GLA_ERR_NO_DEVICE:
        return gpu_adapter_not_found();
    case GLA_ERR_DEVICE:
        return gpu_device_error(m);
    case GLA_ERR_BUFFER:
        return gpu_buffer_error(m);
    case GLA_ERR_POOL_EXHAUSTED:
        return kv_page_pool_exhausted(0, 0, 0);
    case GLA_ERR_KERNEL:
    case GLA_ERR_INVALID:  // an unsupported shape: the caller keeps its CPU path, as for MAX_SEQ
    default:
        return gpu_shader_error(m);
    }
}

std::string GlintError::to_string() const {
    switch (kind_) {
    case Kind::GpuAdapterNotFound:
        return "no compatible GPU adapter found (need a HIP device)";
    case Kind::GpuDeviceError:
        return "GPU device error: " + msg_;
    case Kind::GpuBufferError:
        return "GPU buffer error: " + msg_;
    case Kind::GpuShaderError:
        return "GPU shader error: " + msg_;
    case Kind::SnapshotCacheSizeMismatch:
        return fmt("snapshot cache layer %zu: expected %zu bytes, found %zu", a_, b_, c_);
    case Kind::KvPagePoolExhausted:
        return fmt("KV page pool exhausted: needed %zu page(s), %zu of %zu free", a_, b_, c_);
    }
    return "unknown error";
}

// ---- Device ---------------------------------------------------------------------

Result<std::shared_ptr<Device>> Device::open(int device) {
    gla_ctx *ctx = nullptr;
    const int rc = gla_create(device, &ctx);
    if (rc != GLA_OK) return GlintError::from_status(rc, "gla_create");
    return std::shared_ptr<Device>(new Device(ctx, device));
}

Device::~Device() { gla_destroy(ctx_); }

// ---- f16 / Q8_0 ---------------------------------------------------------------------

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int exp = (h >> 10) & 0x1f;
    const uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);  // inf / nan
    } else if (exp != 0) {
        bits = sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;  // +-0
    } else {          // subnormal: man * 2^-24, exact in f32
        float f = (float)man * 0x1p-24f;
        std::memcpy(&bits, &f, 4);
        bits |= sign;
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

void q8_dequant_range(const uint8_t *row, size_t e0, size_t e1, float *out) {
    for (size_t e = e0; e < e1; e++) {
        const uint8_t *blk = row + (e / 32) * 34;
        const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        out[e - e0] = (float)(int8_t)blk[2 + e % 32] * d;
    }
}

namespace {

// One exported K or V row (f32 bytes or Q8_0 blocks) as kv_dim floats.
void decode_row(const uint8_t *bytes, gla_kv_dtype dtype, size_t kv_dim, float *out) {
    if (dtype == GLA_KV_F32)
        std::memcpy(out, bytes, kv_dim * sizeof(float));
    else
        q8_dequant_range(bytes, 0, kv_dim, out);
}

}  // namespace

// ---- DevicePageStore -------------------------------------------------------------

Result<std::shared_ptr<DevicePageStore>> DevicePageStore::create(std::shared_ptr<Device> dev, gla_kv_dtype dtype,
                                                                 size_t n_kv_heads, size_t head_dim,
                                                                 size_t capacity_pages) {
    gla_kv *kv = nullptr;
    const int rc = gla_pool_create(dev->ctx(), dtype, (int)n_kv_heads, (int)head_dim, (int)capacity_pages, &kv);
    if (rc != GLA_OK) return GlintError::from_status(rc, "gla_pool_create");
    return std::shared_ptr<DevicePageStore>(
        new DevicePageStore(std::move(dev), kv, dtype, n_kv_heads, head_dim, capacity_pages));
}

DevicePageStore::~DevicePageStore() { gla_kv_destroy(kv_); }

size_t DevicePageStore::row_bytes() const { return (size_t)gla_kv_row_bytes(kv_); }

Status DevicePageStore::write_rows(const int64_t *rows, size_t n, const float *k, const float *v) {
    return check(gla_kv_write_rows_host(dev_->ctx(), kv_, rows, k, v, (int)n), "gla_kv_write_rows_host");
}
Status DevicePageStore::export_rows(const int64_t *rows, size_t n, uint8_t *k, uint8_t *v) const {
    return check(gla_kv_export_rows_host(dev_->ctx(), kv_, rows, (int)n, k, v), "gla_kv_export_rows_host");
}
Status DevicePageStore::import_rows(const int64_t *rows, size_t n, const uint8_t *k, const uint8_t *v) {
    return check(gla_kv_import_rows_host(dev_->ctx(), kv_, rows, (int)n, k, v), "gla_kv_import_rows_host");
}
Status DevicePageStore::copy_page(size_t src, size_t dst) {
    return check(gla_pool_copy_page(dev_->ctx(), kv_, (int)src, (int)dst), "gla_pool_copy_page");
}
Status DevicePageStore::zero_page(size_t page) {
    return check(gla_pool_zero_page(dev_->ctx(), kv_, (int)page), "gla_pool_zero_page");
}

// ---- PagePool ---------------------------------------------------------------------

struct PagePool::Inner {
    std::mutex mu;
    std::shared_ptr<PageStore> store;
    size_t capacity = 0;
    size_t live = 0;
    size_t peak_live = 0;
    std::vector<int32_t> free;     // pages to hand out again (LIFO, as Vec::pop)
    int32_t next_fresh = 0;        // pages >= next_fresh were never handed out
    std::vector<uint32_t> refs;    // holders of each page (Arc::strong_count)
    std::vector<uint8_t> dirty;    // returned by a sequence since it was last wiped

    // src/cache/paged.rs:115-125
    Status check_available(size_t n) const {
        if (live + n > capacity) return GlintError::kv_page_pool_exhausted(n, capacity - live, capacity);
        return {};
    }

    // Hand out one page (after check_available). A recycled page is wiped
    // (PageBuf::reset, paged.rs:79-82) unless the caller overwrites all of it.
    Result<int32_t> acquire(bool will_overwrite) {
        int32_t id;
        if (!free.empty()) {
            id = free.back();
            free.pop_back();
        } else {
            id = next_fresh++;
        }
        if (dirty[id] && !will_overwrite) {
            Status s = store->zero_page((size_t)id);
            if (!s) {
                free.push_back(id);
                return s.error();
            }
        }
        dirty[id] = 0;
        refs[id] = 1;
        live += 1;
        peak_live = std::max(peak_live, live);
        return id;
    }

    // Drop one reference; the last holder returns the page (paged.rs:141-151).
    void release(int32_t id) {
        if (--refs[id] == 0) {
            live -= 1;
            free.push_back(id);
            dirty[id] = 1;
        }
    }

    // Replace a shared page with a private copy (paged.rs:427-444).
    Status copy_on_write(int32_t &slot) {
        Result<int32_t> fresh = acquire(true);
        if (!fresh) return fresh.error();
        Status s = store->copy_page((size_t)slot, (size_t)fresh.value());
        if (!s) {
            release(fresh.value());
            return s;
        }
        release(slot);
        slot = fresh.value();
        return {};
    }
};

PagePool::PagePool(std::shared_ptr<PageStore> store) : inner_(std::make_shared<Inner>()) {
    if (!store) throw Panic("PagePool: null page store");
    inner_->capacity = store->capacity();
    inner_->refs.assign(inner_->capacity, 0);
    inner_->dirty.assign(inner_->capacity, 0);
    inner_->store = std::move(store);
}

PagePool PagePool::preallocated(std::shared_ptr<PageStore> store) {
    PagePool pool(std::move(store));
    Inner &in = *pool.inner_;
    in.free.resize(in.capacity);
    std::iota(in.free.begin(), in.free.end(), 0);
    in.next_fresh = (int32_t)in.capacity;
    return pool;
}

size_t PagePool::kv_dim() const { return inner_->store->kv_dim(); }
size_t PagePool::capacity() const { return inner_->capacity; }
size_t PagePool::live_pages() const {
    std::lock_guard<std::mutex> g(inner_->mu);
    return inner_->live;
}
size_t PagePool::available_pages() const {
    std::lock_guard<std::mutex> g(inner_->mu);
    return inner_->capacity - inner_->live;
}
PoolStats PagePool::stats() const {
    std::lock_guard<std::mutex> g(inner_->mu);
    return PoolStats{inner_->capacity, inner_->live, inner_->peak_live, inner_->free.size()};
}
PageStore &PagePool::store() const { return *inner_->store; }
size_t PagePool::refcount(int32_t page) const {
    std::lock_guard<std::mutex> g(inner_->mu);
    return inner_->refs.at((size_t)page);
}

// ---- PagedKvCache -------------------------------------------------------------------

PagedKvCache::PagedKvCache(const PagePool &pool, size_t n_layers) : pool_(pool), table_(n_layers) {}

PagedKvCache::PagedKvCache(const PagePool &pool, std::vector<std::vector<int32_t>> table, size_t len)
    : pool_(pool), table_(std::move(table)), len_(len) {}

PagedKvCache::~PagedKvCache() {
    try {
        release();
    } catch (...) {
    }
}

PagedKvCache::PagedKvCache(PagedKvCache &&o) noexcept : pool_(o.pool_), table_(std::move(o.table_)), len_(o.len_) {
    o.table_.assign(table_.size(), {});
    o.len_ = 0;
}

PagedKvCache &PagedKvCache::operator=(PagedKvCache &&o) noexcept {
    if (this != &o) {
        try {
            release();
        } catch (...) {
        }
        pool_ = o.pool_;
        table_ = std::move(o.table_);
        len_ = o.len_;
        o.table_.assign(table_.size(), {});
        o.len_ = 0;
    }
    return *this;
}

PagedKvCache PagedKvCache::fork_from(size_t upto_position) const {
    if (upto_position > len_) throw Panic(fmt("fork_from: %zu > len %zu", upto_position, len_));
    const size_t pages = div_ceil(upto_position, PAGE_SIZE);
    std::vector<std::vector<int32_t>> t(table_.size());
    std::lock_guard<std::mutex> g(pool_.inner_->mu);
    for (size_t l = 0; l < table_.size(); l++) {
        if (pages > table_[l].size()) throw Panic(fmt("fork_from: layer %zu holds %zu pages < %zu", l,
                                                      table_[l].size(), pages));
        t[l].assign(table_[l].begin(), table_[l].begin() + (ptrdiff_t)pages);
        for (int32_t id : t[l]) pool_.inner_->refs[id] += 1;
    }
    return PagedKvCache(pool_, std::move(t), upto_position);
}

void PagedKvCache::release() {
    if (!pool_.inner_) return;
    std::lock_guard<std::mutex> g(pool_.inner_->mu);
    for (auto &layer : table_) {
        for (int32_t id : layer) pool_.inner_->release(id);
        layer.clear();
    }
    len_ = 0;
}

size_t PagedKvCache::allocated_pages() const {
    size_t n = 0;
    for (const auto &l : table_) n += l.size();
    return n;
}

size_t PagedKvCache::page_refcount(size_t layer, size_t page) const {
    if (layer >= table_.size() || page >= table_[layer].size())
        throw Panic(fmt("page_refcount: (layer %zu, page %zu) not held", layer, page));
    return pool_.refcount(table_[layer][page]);
}

// Grow every layer to cover total_positions and un-share the pages the
// coming appends write into; counts first, so an exhausted pool changes
// nothing (paged.rs:374-411).
Status PagedKvCache::ensure_capacity(size_t total_positions) {
    const size_t want = div_ceil(total_positions, PAGE_SIZE);
    const size_t first_writable = len_ / PAGE_SIZE;
    PagePool::Inner &in = *pool_.inner_;
    std::lock_guard<std::mutex> g(in.mu);
    size_t needed = 0;
    for (const auto &layer : table_) {
        needed += want > layer.size() ? want - layer.size() : 0;
        for (size_t i = first_writable; i < std::min(want, layer.size()); i++) needed += in.refs[layer[i]] > 1;
    }
    if (needed == 0) return {};
    Status s = in.check_available(needed);
    if (!s) return s;
    for (auto &layer : table_) {
        while (layer.size() < want) {
            Result<int32_t> id = in.acquire(false);
            if (!id) return id.error();
            layer.push_back(id.value());
        }
        for (size_t i = first_writable; i < want; i++)
            if (in.refs[layer[i]] > 1) {
                s = in.copy_on_write(layer[i]);
                if (!s) return s;
            }
    }
    return {};
}

// Make pages first_page ..= last_page of `layer` present and private
// (paged.rs:413-435, for a range).
Status PagedKvCache::make_writable(size_t layer, size_t first_page, size_t last_page) {
    PagePool::Inner &in = *pool_.inner_;
    auto &t = table_[layer];
    size_t needed = last_page + 1 > t.size() ? last_page + 1 - t.size() : 0;
    for (size_t i = first_page; i < std::min(last_page + 1, t.size()); i++) needed += in.refs[t[i]] > 1;
    Status s = in.check_available(needed);
    if (!s) return s;
    while (t.size() <= last_page) {
        Result<int32_t> id = in.acquire(false);
        if (!id) return id.error();
        t.push_back(id.value());
    }
    for (size_t i = first_page; i <= last_page; i++)
        if (in.refs[t[i]] > 1) {
            s = in.copy_on_write(t[i]);
            if (!s) return s;
        }
    return {};
}

void PagedKvCache::write(size_t layer, size_t pos, const float *k, const float *v) { write_chunk(layer, pos, 1, k, v); }

void PagedKvCache::write_chunk(size_t layer, size_t pos0, size_t n, const float *k, const float *v) {
    if (n == 0) return;
    if (layer >= table_.size()) throw Panic(fmt("write: layer %zu >= %zu", layer, table_.size()));
    PagePool::Inner &in = *pool_.inner_;
    std::lock_guard<std::mutex> g(in.mu);
    const size_t p0 = pos0 / PAGE_SIZE, p1 = (pos0 + n - 1) / PAGE_SIZE;
    bool private_pages = p1 < table_[layer].size();
    for (size_t i = p0; private_pages && i <= p1; i++) private_pages = in.refs[table_[layer][i]] == 1;
    if (!private_pages) {
        Status s = make_writable(layer, p0, p1);
        if (!s)
            throw Panic(fmt("paged KV-cache write at pos %zu: %s — call KvStore::reserve() before the forward pass "
                            "to handle exhaustion",
                            pos0, s.error().to_string().c_str()));
    }
    std::vector<int64_t> rows(n);
    for (size_t i = 0; i < n; i++) {
        const size_t pos = pos0 + i;
        rows[i] = (int64_t)table_[layer][pos / PAGE_SIZE] * (int64_t)PAGE_SIZE + (int64_t)(pos % PAGE_SIZE);
    }
    Status s = in.store->write_rows(rows.data(), n, k, v);
    if (!s) throw Panic("paged KV-cache write: " + s.error().to_string());
}

std::vector<float> PagedKvCache::row_at(size_t layer, size_t pos, bool want_v) const {
    if (layer >= table_.size() || pos / PAGE_SIZE >= table_[layer].size())
        throw Panic(fmt("paged KV-cache read: (layer %zu, pos %zu) not held", layer, pos));
    PageStore &st = *pool_.inner_->store;
    const int64_t row = (int64_t)table_[layer][pos / PAGE_SIZE] * (int64_t)PAGE_SIZE + (int64_t)(pos % PAGE_SIZE);
    std::vector<uint8_t> kb(st.row_bytes()), vb(st.row_bytes());
    {
        std::lock_guard<std::mutex> g(pool_.inner_->mu);
        Status s = st.export_rows(&row, 1, kb.data(), vb.data());
        if (!s) throw Panic("paged KV-cache read: " + s.error().to_string());
    }
    std::vector<float> out(st.kv_dim());
    decode_row(want_v ? vb.data() : kb.data(), st.dtype(), st.kv_dim(), out.data());
    return out;
}

std::vector<float> PagedKvCache::k_at(size_t layer, size_t pos) const { return row_at(layer, pos, false); }
std::vector<float> PagedKvCache::v_at(size_t layer, size_t pos) const { return row_at(layer, pos, true); }

void PagedKvCache::read_k_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const {
    const std::vector<float> r = row_at(layer, pos, false);
    std::memcpy(buf, r.data() + kv_h * head_dim, head_dim * sizeof(float));
}
void PagedKvCache::read_v_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const {
    const std::vector<float> r = row_at(layer, pos, true);
    std::memcpy(buf, r.data() + kv_h * head_dim, head_dim * sizeof(float));
}

void PagedKvCache::truncate(size_t new_len) {
    if (new_len > len_) throw Panic(fmt("truncate: %zu > len %zu", new_len, len_));
    len_ = new_len;
}

std::pair<std::vector<std::vector<uint8_t>>, std::vector<std::vector<uint8_t>>> PagedKvCache::export_raw() const {
    PageStore &st = *pool_.inner_->store;
    const size_t rb = st.row_bytes();
    std::vector<std::vector<uint8_t>> ko(table_.size()), vo(table_.size());
    std::vector<int64_t> rows(len_);
    for (size_t l = 0; l < table_.size(); l++) {
        for (size_t pos = 0; pos < len_; pos++)
            rows[pos] = (int64_t)table_[l].at(pos / PAGE_SIZE) * (int64_t)PAGE_SIZE + (int64_t)(pos % PAGE_SIZE);
        ko[l].resize(len_ * rb);
        vo[l].resize(len_ * rb);
        std::lock_guard<std::mutex> g(pool_.inner_->mu);
        Status s = st.export_rows(rows.data(), len_, ko[l].data(), vo[l].data());
        if (!s) throw Panic("paged KV-cache export: " + s.error().to_string());
    }
    return {std::move(ko), std::move(vo)};
}

Status PagedKvCache::import_raw(const std::vector<std::vector<uint8_t>> &k_layers,
                                const std::vector<std::vector<uint8_t>> &v_layers, size_t token_count) {
    PageStore &st = *pool_.inner_->store;
    const size_t expected = token_count * st.row_bytes();
    const size_t n = std::min(k_layers.size(), v_layers.size());
    for (size_t l = 0; l < n; l++) {
        if (k_layers[l].size() != expected)
            return GlintError::snapshot_cache_size_mismatch(l, expected, k_layers[l].size());
        if (v_layers[l].size() != expected)
            return GlintError::snapshot_cache_size_mismatch(l, expected, v_layers[l].size());
    }
    // pages for the whole snapshot first: a pool that cannot hold it fails here
    len_ = 0;
    Status s = ensure_capacity(token_count);
    if (!s) return s;
    std::vector<int64_t> rows(token_count);
    for (size_t l = 0; l < n; l++) {
        if (l >= table_.size()) throw Panic(fmt("import_raw: layer %zu >= %zu", l, table_.size()));
        for (size_t pos = 0; pos < token_count; pos++)
            rows[pos] = (int64_t)table_[l][pos / PAGE_SIZE] * (int64_t)PAGE_SIZE + (int64_t)(pos % PAGE_SIZE);
        std::lock_guard<std::mutex> g(pool_.inner_->mu);
        s = st.import_rows(rows.data(), token_count, k_layers[l].data(), v_layers[l].data());
        if (!s) return s;
    }
    len_ = token_count;
    return {};
}

// ---- GpuKvCache ------------------------------------------------------------------------

class GpuKvStorage {
  public:
    GpuKvStorage(std::shared_ptr<Device> dev, gla_kv *kv, gla_kv_dtype dtype, size_t n_seqs, size_t n_layers,
                 size_t max_seq_len, size_t n_kv_heads, size_t head_dim)
        : dev(std::move(dev)), kv(kv), dtype(dtype), n_seqs(n_seqs), n_layers(n_layers), max_seq_len(max_seq_len),
          n_kv_heads(n_kv_heads), head_dim(head_dim), row_bytes((size_t)gla_kv_row_bytes(kv)) {}
    ~GpuKvStorage() { gla_kv_destroy(kv); }
    GpuKvStorage(const GpuKvStorage &) = delete;
    GpuKvStorage &operator=(const GpuKvStorage &) = delete;
    int64_t row(int seq, size_t layer, size_t pos) const { return gla_kv_row_id(kv, seq, (int)layer, (int)pos); }

    std::shared_ptr<Device> dev;
    gla_kv *kv;
    gla_kv_dtype dtype;
    size_t n_seqs, n_layers, max_seq_len, n_kv_heads, head_dim, row_bytes;
};

GpuKvCache::GpuKvCache(std::shared_ptr<GpuKvStorage> storage, int seq) : storage_(std::move(storage)) {
    buf_.kv = storage_->kv;
    buf_.seq = seq;
    buf_.n_layers = storage_->n_layers;
    buf_.n_kv_heads = storage_->n_kv_heads;
    buf_.head_dim = storage_->head_dim;
    buf_.max_seq_len = storage_->max_seq_len;
}

size_t GpuKvCache::kv_dim() const { return storage_->n_kv_heads * storage_->head_dim; }
size_t GpuKvCache::max_seq_len() const { return storage_->max_seq_len; }
gla_kv_dtype GpuKvCache::dtype() const { return storage_->dtype; }

void GpuKvCache::write(size_t layer, size_t pos, const float *k, const float *v) { write_chunk(layer, pos, 1, k, v); }

void GpuKvCache::write_chunk(size_t layer, size_t pos0, size_t n, const float *k, const float *v) {
    if (n == 0) return;
    if (pos0 + n > storage_->max_seq_len)
        throw Panic(fmt("KV-cache overflow: pos %zu >= %zu", pos0 + n - 1, storage_->max_seq_len));
    if (layer >= storage_->n_layers) throw Panic(fmt("write: layer %zu >= %zu", layer, storage_->n_layers));
    std::vector<int64_t> rows(n);
    for (size_t i = 0; i < n; i++) rows[i] = storage_->row(buf_.seq, layer, pos0 + i);
    Status s = check(gla_kv_write_rows_host(storage_->dev->ctx(), storage_->kv, rows.data(), k, v, (int)n),
                     "gla_kv_write_rows_host");
    if (!s) throw Panic("KV-cache write: " + s.error().to_string());
}

std::vector<float> GpuKvCache::row_at(size_t layer, size_t pos, bool want_v) const {
    if (layer >= storage_->n_layers || pos >= storage_->max_seq_len)
        throw Panic(fmt("KV-cache read: (layer %zu, pos %zu) out of range", layer, pos));
    const int64_t row = storage_->row(buf_.seq, layer, pos);
    std::vector<uint8_t> kb(storage_->row_bytes), vb(storage_->row_bytes);
    Status s = check(gla_kv_export_rows_host(storage_->dev->ctx(), storage_->kv, &row, 1, kb.data(), vb.data()),
                     "gla_kv_export_rows_host");
    if (!s) throw Panic("KV-cache read: " + s.error().to_string());
    std::vector<float> out(kv_dim());
    decode_row(want_v ? vb.data() : kb.data(), storage_->dtype, kv_dim(), out.data());
    return out;
}

std::vector<float> GpuKvCache::k_at(size_t layer, size_t pos) const { return row_at(layer, pos, false); }
std::vector<float> GpuKvCache::v_at(size_t layer, size_t pos) const { return row_at(layer, pos, true); }

void GpuKvCache::read_k_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const {
    const std::vector<float> r = row_at(layer, pos, false);
    std::memcpy(buf, r.data() + kv_h * head_dim, head_dim * sizeof(float));
}
void GpuKvCache::read_v_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const {
    const std::vector<float> r = row_at(layer, pos, true);
    std::memcpy(buf, r.data() + kv_h * head_dim, head_dim * sizeof(float));
}

void GpuKvCache::truncate(size_t new_len) {
    if (new_len > len_) throw Panic(fmt("truncate: %zu > len %zu", new_len, len_));
    len_ = new_len;
}

std::pair<std::vector<std::vector<uint8_t>>, std::vector<std::vector<uint8_t>>> GpuKvCache::export_raw() const {
    const size_t rb = storage_->row_bytes;
    std::vector<std::vector<uint8_t>> ko(storage_->n_layers), vo(storage_->n_layers);
    std::vector<int64_t> rows(len_);
    for (size_t l = 0; l < storage_->n_layers; l++) {
        for (size_t pos = 0; pos < len_; pos++) rows[pos] = storage_->row(buf_.seq, l, pos);
        ko[l].resize(len_ * rb);
        vo[l].resize(len_ * rb);
        Status s = check(gla_kv_export_rows_host(storage_->dev->ctx(), storage_->kv, rows.data(), (int)len_,
                                                 ko[l].data(), vo[l].data()),
                         "gla_kv_export_rows_host");
        if (!s) throw Panic("KV-cache export: " + s.error().to_string());
    }
    return {std::move(ko), std::move(vo)};
}

// KvCache::import_raw (src/cache/mod.rs:211-258): layer by layer, each
// checked and then copied.
Status GpuKvCache::import_raw(const std::vector<std::vector<uint8_t>> &k_layers,
                              const std::vector<std::vector<uint8_t>> &v_layers, size_t token_count) {
    const size_t expected = token_count * storage_->row_bytes;
    const size_t n = std::min(k_layers.size(), v_layers.size());
    std::vector<int64_t> rows(token_count);
    for (size_t l = 0; l < n; l++) {
        if (k_layers[l].size() != expected)
            return GlintError::snapshot_cache_size_mismatch(l, expected, k_layers[l].size());
        if (v_layers[l].size() != expected)
            return GlintError::snapshot_cache_size_mismatch(l, expected, v_layers[l].size());
        if (l >= storage_->n_layers || token_count > storage_->max_seq_len)
            throw Panic(fmt("import_raw: layer %zu / %zu positions outside the cache", l, token_count));
        for (size_t pos = 0; pos < token_count; pos++) rows[pos] = storage_->row(buf_.seq, l, pos);
        Status s = check(gla_kv_import_rows_host(storage_->dev->ctx(), storage_->kv, rows.data(), (int)token_count,
                                                 k_layers[l].data(), v_layers[l].data()),
                         "gla_kv_import_rows_host");
        if (!s) return s;
    }
    len_ = token_count;
    return {};
}

// ---- GpuBackend -------------------------------------------------------------------------

// Device buffers for the batched calls, grown on demand and reused.
struct GpuBackend::Staging {
    explicit Staging(std::shared_ptr<Device> d) : dev(std::move(d)) {}
    ~Staging() {
        for (auto &b : bufs)
            if (b.ptr) gla_dev_free(dev->ctx(), b.ptr);
    }
    struct Buf {
        void *ptr = nullptr;
        size_t bytes = 0;
    };
    enum { Q, OUT, TABLE, START, LEN, SLOT, QSTART, POSOFF, POS, N_BUFS };
    std::shared_ptr<Device> dev;
    Buf bufs[N_BUFS];

    Result<void *> get(int which, size_t bytes) {
        Buf &b = bufs[which];
        if (b.bytes < bytes) {
            if (b.ptr) gla_dev_free(dev->ctx(), b.ptr);
            b.ptr = nullptr;
            b.bytes = 0;
            const size_t want = std::max<size_t>(bytes, 256);
            const int rc = gla_dev_alloc(dev->ctx(), want, &b.ptr);
            if (rc != GLA_OK) return GlintError::from_status(rc, "gla_dev_alloc");
            b.bytes = want;
        }
        return b.ptr;
    }
    // Upload host bytes into buffer `which`.
    Result<void *> put(int which, const void *src, size_t bytes) {
        Result<void *> p = get(which, bytes);
        if (!p) return p;
        if (bytes) {
            const int rc = gla_memcpy_htod(dev->ctx(), p.value(), src, bytes);
            if (rc != GLA_OK) return GlintError::from_status(rc, "gla_memcpy_htod");
        }
        return p;
    }
};

Result<GpuBackend> GpuBackend::create(int device) {
    Result<std::shared_ptr<Device>> d = Device::open(device);
    if (!d) return d.error();
    return GpuBackend(std::move(d).value());
}

GpuBackend::GpuBackend(std::shared_ptr<Device> dev) : dev_(std::move(dev)), stage_(new Staging(dev_)) {}
GpuBackend::GpuBackend(GpuBackend &&) noexcept = default;
GpuBackend &GpuBackend::operator=(GpuBackend &&) noexcept = default;
GpuBackend::~GpuBackend() = default;

gla_ctx *GpuBackend::ctx() const { return dev_->ctx(); }

std::string GpuBackend::info_string() const {
    return fmt("HIP device %d (gfx950 attention, %d CUs)", dev_->ordinal(), gla_device_cu_count(dev_->ctx()));
}

Result<std::vector<float>> GpuBackend::attention(const std::vector<float> &q, const std::vector<float> &k,
                                                 const std::vector<float> &v, uint32_t n_heads, uint32_t n_kv_heads,
                                                 uint32_t head_dim, uint32_t seq_len, float scale, float softcap) {
    const size_t kv_dim = (size_t)n_kv_heads * head_dim;
    if (q.size() != (size_t)n_heads * head_dim || k.size() < (size_t)seq_len * kv_dim ||
        v.size() < (size_t)seq_len * kv_dim)
        return GlintError::gpu_buffer_error("attention: slice lengths do not match the shape");
    std::vector<float> out((size_t)n_heads * head_dim);
    Status s = check(gla_attention(dev_->ctx(), q.data(), k.data(), v.data(), (int)n_heads, (int)n_kv_heads,
                                   (int)head_dim, (int)seq_len, scale, softcap, out.data()),
                     "gla_attention");
    if (!s) return s.error();
    return out;
}

Result<std::vector<float>> GpuBackend::attention_resident(const std::vector<float> &q, const GpuKvBuffer &kv_buf,
                                                          size_t layer_idx, size_t window_start, size_t attend_len,
                                                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                                          float scale, float softcap) {
    if (!kv_buf.kv || kv_buf.n_kv_heads != n_kv_heads || kv_buf.head_dim != head_dim)
        return GlintError::gpu_shader_error("attention_resident: shape does not match the cache");
    if (q.size() != (size_t)n_heads * head_dim)
        return GlintError::gpu_buffer_error("attention_resident: q length does not match the shape");
    if (layer_idx >= kv_buf.n_layers)
        return GlintError::gpu_shader_error(fmt("attention_resident: layer %zu >= %zu", layer_idx, kv_buf.n_layers));
    std::vector<float> out((size_t)n_heads * head_dim);
    Status s = check(gla_attention_resident(dev_->ctx(), q.data(), kv_buf.kv, kv_buf.seq, (int)layer_idx,
                                            (int)window_start, (int)attend_len, (int)n_heads, scale, softcap,
                                            out.data()),
                     "gla_attention_resident");
    if (!s) return s.error();
    return out;
}

Result<GpuKvCache> GpuBackend::create_kv_cache(size_t n_layers, size_t max_seq_len, size_t n_kv_heads,
                                               size_t head_dim, gla_kv_dtype dtype) {
    Result<std::vector<GpuKvCache>> v = create_kv_caches(1, n_layers, max_seq_len, n_kv_heads, head_dim, dtype);
    if (!v) return v.error();
    return std::move(v.value()[0]);
}

Result<std::vector<GpuKvCache>> GpuBackend::create_kv_caches(size_t n_seqs, size_t n_layers, size_t max_seq_len,
                                                             size_t n_kv_heads, size_t head_dim,
                                                             gla_kv_dtype dtype) {
    gla_kv *kv = nullptr;
    const int rc = gla_kv_cache_create(dev_->ctx(), dtype, (int)n_seqs, (int)n_layers, (int)max_seq_len,
                                       (int)n_kv_heads, (int)head_dim, &kv);
    if (rc != GLA_OK) return GlintError::from_status(rc, "gla_kv_cache_create");
    auto st = std::make_shared<GpuKvStorage>(dev_, kv, dtype, n_seqs, n_layers, max_seq_len, n_kv_heads, head_dim);
    std::vector<GpuKvCache> out;
    out.reserve(n_seqs);
    for (size_t s = 0; s < n_seqs; s++) out.emplace_back(st, (int)s);
    return out;
}

Result<PagePool> GpuBackend::create_page_pool(size_t capacity_pages, size_t n_kv_heads, size_t head_dim,
                                              gla_kv_dtype dtype) {
    Result<std::shared_ptr<DevicePageStore>> st =
        DevicePageStore::create(dev_, dtype, n_kv_heads, head_dim, capacity_pages);
    if (!st) return st.error();
    return PagePool::preallocated(std::move(st).value());
}

namespace {

// What one launch reads: a device page pool or one contiguous storage.
struct Source {
    const gla_kv *kv = nullptr;
    bool paged = false;
    size_t kv_dim = 0;
};

Result<Source> source_of(const std::vector<const KvStore *> &stores, const char *what) {
    Source src;
    for (size_t i = 0; i < stores.size(); i++) {
        const KvStore *s = stores[i];
        if (!s) return GlintError::gpu_shader_error(fmt("%s: cache %zu is null", what, i));
        const gla_kv *kv;
        bool paged;
        size_t kv_dim;
        if (const PagedKvCache *p = s->as_paged()) {
            kv = p->pool().store().device_kv();
            paged = true;
            kv_dim = p->pool().kv_dim();
        } else if (const GpuKvBuffer *b = s->gpu_buffer()) {
            kv = b->kv;
            paged = false;
            kv_dim = b->n_kv_heads * b->head_dim;
        } else {
            kv = nullptr;
            paged = false;
            kv_dim = 0;
        }
        if (!kv) return GlintError::gpu_shader_error(fmt("%s: cache %zu is not device-resident", what, i));
        if (i == 0) {
            src = Source{kv, paged, kv_dim};
        } else if (kv != src.kv) {
            return GlintError::gpu_shader_error(fmt("%s: caches must share one device storage or page pool", what));
        }
    }
    return src;
}

}  // namespace

Result<std::vector<float>> GpuBackend::decode_batch(const std::vector<DecodeSeq> &seqs, const float *q,
                                                    size_t layer, const AttnShape &shape) {
    const size_t B = seqs.size();
    const size_t row = (size_t)shape.n_heads * shape.head_dim;
    if (B == 0) return std::vector<float>();
    std::vector<const KvStore *> stores(B);
    for (size_t b = 0; b < B; b++) stores[b] = seqs[b].kv;
    Result<Source> src = source_of(stores, "decode_batch");
    if (!src) return src.error();
    const Source &S = src.value();
    if (S.kv_dim != (size_t)shape.n_kv_heads * shape.head_dim)
        return GlintError::gpu_shader_error("decode_batch: n_kv_heads * head_dim does not match the cache");
    std::vector<int32_t> start(B), len(B), slot;
    std::vector<int32_t> table;
    int stride = 0;
    int max_len = 0;
    for (size_t b = 0; b < B; b++) {
        const size_t end = seqs[b].window_start + seqs[b].attend_len;
        if (S.paged) {
            const PagedKvCache *p = seqs[b].kv->as_paged();
            if (layer >= p->n_layers()) return GlintError::gpu_shader_error("decode_batch: layer out of range");
            if (div_ceil(end, PAGE_SIZE) > p->page_table(layer).size())
                return GlintError::gpu_shader_error(fmt("decode_batch: sequence %zu attends positions to %zu but "
                                                        "holds %zu pages", b, end, p->page_table(layer).size()));
            stride = std::max(stride, (int)p->page_table(layer).size());
        } else {
            const GpuKvBuffer *g = seqs[b].kv->gpu_buffer();
            if (layer >= g->n_layers) return GlintError::gpu_shader_error("decode_batch: layer out of range");
            if (end > g->max_seq_len)
                return GlintError::gpu_shader_error(fmt("decode_batch: window end %zu > max_seq_len %zu", end,
                                                        g->max_seq_len));
            slot.push_back(g->seq);
        }
        start[b] = (int32_t)seqs[b].window_start;
        len[b] = (int32_t)seqs[b].attend_len;
        max_len = std::max(max_len, len[b]);
    }
    gla_decode_args a{};
    a.kv = S.kv;
    a.layer = (int)layer;
    a.n_seqs = (int)B;
    Staging &st = *stage_;
    Result<void *> p = st.put(Staging::Q, q, B * row * sizeof(float));
    if (!p) return p.error();
    a.q = (const float *)p.value();
    if (!(p = st.get(Staging::OUT, B * row * sizeof(float)))) return p.error();
    a.out = (float *)p.value();
    if (!(p = st.put(Staging::START, start.data(), B * 4))) return p.error();
    a.kv_start = (const int32_t *)p.value();
    if (!(p = st.put(Staging::LEN, len.data(), B * 4))) return p.error();
    a.kv_len = (const int32_t *)p.value();
    if (S.paged) {
        stride = std::max(stride, 1);
        table.assign(B * (size_t)stride, 0);
        for (size_t b = 0; b < B; b++) {
            const auto &t = seqs[b].kv->as_paged()->page_table(layer);
            std::copy(t.begin(), t.end(), table.begin() + (ptrdiff_t)(b * stride));
        }
        if (!(p = st.put(Staging::TABLE, table.data(), table.size() * 4))) return p.error();
        a.page_table = (const int32_t *)p.value();
        a.page_table_stride = stride;
    } else {
        if (!(p = st.put(Staging::SLOT, slot.data(), B * 4))) return p.error();
        a.seq_slot = (const int32_t *)p.value();
    }
    a.max_kv_len = max_len;
    a.n_heads = (int)shape.n_heads;
    a.scale = shape.scale;
    a.softcap = shape.softcap;
    a.kv_start_host = start.data();
    a.kv_len_host = len.data();
    Status s = check(gla_decode(dev_->ctx(), &a), "gla_decode");
    if (!s) return s.error();
    std::vector<float> out(B * row);
    s = check(gla_memcpy_dtoh(dev_->ctx(), out.data(), a.out, out.size() * sizeof(float)), "gla_memcpy_dtoh");
    if (!s) return s.error();
    return out;
}

Result<std::vector<float>> GpuBackend::prefill_batch(const std::vector<PrefillSeq> &seqs, const float *q,
                                                     size_t layer, const AttnShape &shape, size_t sliding_window,
                                                     gla_precision precision) {
    const size_t B = seqs.size();
    const size_t row = (size_t)shape.n_heads * shape.head_dim;
    if (B == 0) return std::vector<float>();
    std::vector<const KvStore *> stores(B);
    for (size_t b = 0; b < B; b++) stores[b] = seqs[b].kv;
    Result<Source> src = source_of(stores, "prefill_batch");
    if (!src) return src.error();
    const Source &S = src.value();
    if (S.kv_dim != (size_t)shape.n_kv_heads * shape.head_dim)
        return GlintError::gpu_shader_error("prefill_batch: n_kv_heads * head_dim does not match the cache");
    std::vector<int32_t> q_start(B + 1, 0), pos_off(B), slot, table;
    int stride = 0, max_q = 0;
    for (size_t b = 0; b < B; b++) {
        const size_t end = seqs[b].pos_offset + seqs[b].n_rows;
        if (S.paged) {
            const PagedKvCache *pc = seqs[b].kv->as_paged();
            if (layer >= pc->n_layers()) return GlintError::gpu_shader_error("prefill_batch: layer out of range");
            if (div_ceil(end, PAGE_SIZE) > pc->page_table(layer).size())
                return GlintError::gpu_shader_error(fmt("prefill_batch: sequence %zu needs positions to %zu", b, end));
            stride = std::max(stride, (int)pc->page_table(layer).size());
        } else {
            const GpuKvBuffer *g = seqs[b].kv->gpu_buffer();
            if (layer >= g->n_layers) return GlintError::gpu_shader_error("prefill_batch: layer out of range");
            if (end > g->max_seq_len)
                return GlintError::gpu_shader_error(fmt("prefill_batch: positions to %zu > max_seq_len %zu", end,
                                                        g->max_seq_len));
            slot.push_back(g->seq);
        }
        q_start[b + 1] = q_start[b] + (int32_t)seqs[b].n_rows;
        pos_off[b] = (int32_t)seqs[b].pos_offset;
        max_q = std::max(max_q, (int)seqs[b].n_rows);
    }
    const size_t rows = (size_t)q_start[B];
    if (rows == 0) return std::vector<float>();
    gla_prefill_args a{};
    a.kv = S.kv;
    a.layer = (int)layer;
    a.n_seqs = (int)B;
    Staging &st = *stage_;
    Result<void *> p = st.put(Staging::Q, q, rows * row * sizeof(float));
    if (!p) return p.error();
    a.q = (const float *)p.value();
    if (!(p = st.get(Staging::OUT, rows * row * sizeof(float)))) return p.error();
    a.out = (float *)p.value();
    if (!(p = st.put(Staging::QSTART, q_start.data(), (B + 1) * 4))) return p.error();
    a.q_start = (const int32_t *)p.value();
    if (!(p = st.put(Staging::POSOFF, pos_off.data(), B * 4))) return p.error();
    a.pos_offset = (const int32_t *)p.value();
    if (S.paged) {
        stride = std::max(stride, 1);
        table.assign(B * (size_t)stride, 0);
        for (size_t b = 0; b < B; b++) {
            const auto &t = seqs[b].kv->as_paged()->page_table(layer);
            std::copy(t.begin(), t.end(), table.begin() + (ptrdiff_t)(b * stride));
        }
        if (!(p = st.put(Staging::TABLE, table.data(), table.size() * 4))) return p.error();
        a.page_table = (const int32_t *)p.value();
        a.page_table_stride = stride;
    } else {
        if (!(p = st.put(Staging::SLOT, slot.data(), B * 4))) return p.error();
        a.seq_slot = (const int32_t *)p.value();
    }
    a.max_q_len = max_q;
    a.n_heads = (int)shape.n_heads;
    a.scale = shape.scale;
    a.softcap = shape.softcap;
    a.sliding_window = (int)sliding_window;
    a.precision = precision;
    Status s = check(gla_prefill(dev_->ctx(), &a), "gla_prefill");
    if (!s) return s.error();
    std::vector<float> out(rows * row);
    s = check(gla_memcpy_dtoh(dev_->ctx(), out.data(), a.out, out.size() * sizeof(float)), "gla_memcpy_dtoh");
    if (!s) return s.error();
    return out;
}

// ---- the ops beside attention ------------------------------------------------------------

GpuQ8Weights::GpuQ8Weights(std::shared_ptr<Device> dev, gla_q8w *w, size_t rows, size_t cols)
    : dev_(std::move(dev)), w_(w), rows_(rows), cols_(cols) {}
GpuQ8Weights::GpuQ8Weights(GpuQ8Weights &&o) noexcept
    : dev_(std::move(o.dev_)), w_(o.w_), rows_(o.rows_), cols_(o.cols_) {
    o.w_ = nullptr;
}
GpuQ8Weights &GpuQ8Weights::operator=(GpuQ8Weights &&o) noexcept {
    if (this != &o) {
        if (w_) gla_q8w_destroy(w_);
        dev_ = std::move(o.dev_);
        w_ = o.w_;
        rows_ = o.rows_;
        cols_ = o.cols_;
        o.w_ = nullptr;
    }
    return *this;
}
GpuQ8Weights::~GpuQ8Weights() {
    if (w_) gla_q8w_destroy(w_);
}

Result<GpuQ8Weights> GpuBackend::upload_q8_0(const uint8_t *ggml, size_t n_bytes, size_t rows, size_t cols) {
    if (cols % 32 != 0 || rows == 0 || cols == 0 || rows > INT32_MAX || cols > INT32_MAX)
        return GlintError::gpu_buffer_error(fmt("upload_q8_0: %zu x %zu is not a Q8_0 matrix", rows, cols));
    if (n_bytes != rows * (cols / 32) * 34)
        return GlintError::gpu_buffer_error(
            fmt("upload_q8_0: %zu bytes for %zu x %zu (expected %zu)", n_bytes, rows, cols, rows * (cols / 32) * 34));
    gla_q8w *w = nullptr;
    Status s = check(gla_q8w_create(dev_->ctx(), ggml, (int)rows, (int)cols, &w), "gla_q8w_create");
    if (!s) return s.error();
    return GpuQ8Weights(dev_, w, rows, cols);
}

Result<std::vector<float>> GpuBackend::matvec_q8_0(const GpuQ8Weights &w, const float *x, size_t n_vec) {
    if (!w.handle()) return GlintError::gpu_shader_error("matvec_q8_0: weights not uploaded");
    if (n_vec == 0) return std::vector<float>();
    if (n_vec > INT32_MAX) return GlintError::gpu_shader_error("matvec_q8_0: too many vectors");
    Staging &st = *stage_;
    Result<void *> px = st.put(Staging::Q, x, n_vec * w.cols() * sizeof(float));
    if (!px) return px.error();
    Result<void *> py = st.get(Staging::OUT, n_vec * w.rows() * sizeof(float));
    if (!py) return py.error();
    Status s = check(gla_matvec_q8_0(dev_->ctx(), w.handle(), (const float *)px.value(), (int)n_vec,
                                     (float *)py.value()),
                     "gla_matvec_q8_0");
    if (!s) return s.error();
    std::vector<float> y(n_vec * w.rows());
    s = check(gla_memcpy_dtoh(dev_->ctx(), y.data(), py.value(), y.size() * sizeof(float)), "gla_memcpy_dtoh");
    if (!s) return s.error();
    return y;
}

Status GpuBackend::rope(float *x, size_t n_rows, size_t n_heads, size_t head_dim, const int32_t *pos,
                        float freq_base, float scaling_factor, size_t rot_dim) {
    if (n_rows == 0) return {};
    if (n_rows > INT32_MAX || n_heads > INT32_MAX || head_dim > INT32_MAX)
        return GlintError::gpu_shader_error("rope: shape out of range");
    const size_t bytes = n_rows * n_heads * head_dim * sizeof(float);
    Staging &st = *stage_;
    Result<void *> px = st.put(Staging::Q, x, bytes);
    if (!px) return px.error();
    Result<void *> pp = st.put(Staging::POS, pos, n_rows * sizeof(int32_t));
    if (!pp) return pp.error();
    Status s = check(gla_rope(dev_->ctx(), (float *)px.value(), (int)n_rows, (int)n_heads, (int)head_dim,
                              (const int32_t *)pp.value(), freq_base, scaling_factor,
                              (int)std::min<size_t>(rot_dim, INT32_MAX)),
                     "gla_rope");
    if (!s) return s;
    return check(gla_memcpy_dtoh(dev_->ctx(), x, px.value(), bytes), "gla_memcpy_dtoh");
}

size_t window_start(size_t pos, size_t sliding_window, bool alternating, size_t layer) {
    return (size_t)gla_window_start((long)pos, (long)sliding_window, alternating ? 1 : 0, (int)layer);
}

}  // namespace glint
