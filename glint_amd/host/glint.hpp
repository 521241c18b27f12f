// glint.hpp -- C++ host layer of the MI355X attention path: the types the
// Rust engine uses around attention (GlintError, KvStore, PagePool,
// PagedKvCache, GpuKvCache, GpuBackend), restated in C++ over the C ABI of
// include/glint_attn.h, with the same names, argument meaning and error
// behaviour:
//   GlintError / Result           src/error.rs:41-52, :69-82, :150-210
//   KvStore                       src/cache/mod.rs:24-109
//   PagePool / PagedKvCache       src/cache/paged.rs:55-598
//   GpuKvBuffer / GpuKvCache      src/backend/gpu.rs:1005-1104, src/cache/mod.rs:430-578
//   GpuBackend::attention{,_resident}, create_kv_cache
//                                 src/backend/gpu.rs:41-56, :266-397, :860-992, :1058-1104
//   batched decode / prefill attention steps
//                                 src/transformer/forward.rs:1468-1507, :879-976
//
// K/V live in HBM. A PagedKvCache keeps its page tables and reference counts
// on the host (one table per layer of device page ids), as PagedKvCache keeps
// Arc<PageBuf>s; the pages themselves are rows of a device pool
// (gla_pool_create), written, copied on write and wiped on recycle by the
// library's kernels. Rust's Result<T, GlintError> is Result<T> here; Rust
// panics (a write past the pool with no reserve, fork_from / truncate past
// len) throw glint::Panic with the reference's message.
//
// Threading: a GpuBackend, and every cache created from it, shares one
// gla_ctx, which is not thread-safe. PagePool serialises its own device work
// (page writes, copies, wipes) under its mutex; callers that drive one
// backend from several threads lock around it, as Glint's single engine
// thread does (src/server/engine.rs:449-459).
#ifndef GLINT_HOST_HPP
#define GLINT_HOST_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <variant>
#include <vector>

#include "glint_attn.h"

namespace glint {

// Positions stored in one page (src/cache/paged.rs:55).
constexpr size_t PAGE_SIZE = GLA_PAGE_SIZE;

// ---- errors ----------------------------------------------------------------

// The GlintError variants this path reports (src/error.rs:41-52, :69-82).
class GlintError {
  public:
    enum class Kind {
        GpuAdapterNotFound,
        GpuDeviceError,
        GpuBufferError,
        GpuShaderError,
        SnapshotCacheSizeMismatch,
        KvPagePoolExhausted,
    };

    static GlintError gpu_adapter_not_found();
    static GlintError gpu_device_error(std::string msg);
    static GlintError gpu_buffer_error(std::string msg);
    static GlintError gpu_shader_error(std::string msg);
    static GlintError snapshot_cache_size_mismatch(size_t layer, size_t expected, size_t found);
    static GlintError kv_page_pool_exhausted(size_t needed, size_t available, size_t capacity);
    // A failed C-ABI call: the status code's variant with gla_last_error()'s text.
    static GlintError from_status(int status, const char *what);

    Kind kind() const { return kind_; }
    const std::string &message() const { return msg_; }
    // KvPagePoolExhausted fields
    size_t needed() const { return a_; }
    size_t available() const { return b_; }
    size_t capacity() const { return c_; }
    // SnapshotCacheSizeMismatch fields
    size_t layer() const { return a_; }
    size_t expected() const { return b_; }
    size_t found() const { return c_; }
    // The Display text of the variant (src/error.rs:150-210).
    std::string to_string() const;

  private:
    GlintError(Kind k, std::string msg, size_t a = 0, size_t b = 0, size_t c = 0)
        : kind_(k), msg_(std::move(msg)), a_(a), b_(b), c_(c) {}
    Kind kind_;
    std::string msg_;
    size_t a_, b_, c_;
};

// A Rust panic on this path (an overflowing write, fork_from or truncate past
// len, unwrap of an error).
class Panic : public std::logic_error {
  public:
    explicit Panic(const std::string &what) : std::logic_error(what) {}
};

// Result<T, GlintError>.
template <class T>
class Result {
  public:
    Result(T value) : v_(std::move(value)) {}
    Result(GlintError err) : v_(std::move(err)) {}
    bool ok() const { return v_.index() == 0; }
    explicit operator bool() const { return ok(); }
    const GlintError &error() const { return std::get<1>(v_); }
    T &value() & {
        if (!ok()) throw Panic("called `Result::unwrap()` on an `Err` value: " + error().to_string());
        return std::get<0>(v_);
    }
    T &&value() && {
        if (!ok()) throw Panic("called `Result::unwrap()` on an `Err` value: " + error().to_string());
        return std::get<0>(std::move(v_));
    }
    T expect(const std::string &what) && {
        if (!ok()) throw Panic(what + ": " + error().to_string());
        return std::get<0>(std::move(v_));
    }

  private:
    std::variant<T, GlintError> v_;
};

template <>
class Result<void> {
  public:
    Result() = default;
    Result(GlintError err) : e_(std::move(err)) {}
    bool ok() const { return !e_.has_value(); }
    explicit operator bool() const { return ok(); }
    const GlintError &error() const { return *e_; }
    void value() const {
        if (!ok()) throw Panic("called `Result::unwrap()` on an `Err` value: " + e_->to_string());
    }
    void expect(const std::string &what) const {
        if (!ok()) throw Panic(what + ": " + e_->to_string());
    }

  private:
    std::optional<GlintError> e_;
};

using Status = Result<void>;

// ---- device ------------------------------------------------------------------

// An open gla_ctx, shared by a backend and the storage created from it.
class Device {
  public:
    static Result<std::shared_ptr<Device>> open(int device);
    ~Device();
    Device(const Device &) = delete;
    Device &operator=(const Device &) = delete;
    gla_ctx *ctx() const { return ctx_; }
    int ordinal() const { return ordinal_; }

  private:
    Device(gla_ctx *ctx, int ordinal) : ctx_(ctx), ordinal_(ordinal) {}
    gla_ctx *ctx_;
    int ordinal_;
};

// ---- KvStore -----------------------------------------------------------------

class PagedKvCache;

// A device-resident contiguous cache as gla_decode reads it: slot `seq` of a
// storage holding several sequences (src/backend/gpu.rs:1011-1027).
struct GpuKvBuffer {
    const gla_kv *kv = nullptr;
    int seq = 0;
    size_t n_layers = 0;
    size_t n_kv_heads = 0;
    size_t head_dim = 0;
    size_t max_seq_len = 0;
};

// src/cache/mod.rs:24-109.
class KvStore {
  public:
    virtual ~KvStore() = default;
    // Fill buf[0 .. head_dim) with the K (V) vector of head kv_h at (layer, pos).
    virtual void read_k_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const = 0;
    virtual void read_v_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const = 0;
    // K and V of one position (all KV heads, kv_dim floats each) in one layer.
    virtual void write(size_t layer, size_t pos, const float *k, const float *v) = 0;
    // Make positions 0 .. total_positions writable; pre-allocated caches
    // already are (mod.rs:35-47).
    virtual Status reserve(size_t total_positions) {
        (void)total_positions;
        return {};
    }
    virtual void advance() = 0;
    virtual size_t len() const = 0;
    bool is_empty() const { return len() == 0; }
    virtual void truncate(size_t new_len) = 0;
    void clear() { truncate(0); }
    // Positions 0 .. len() as bytes, one vector per layer: native f32 rows, or
    // Q8_0 rows of ceil(kv_dim/32) x [f16 scale LE][32 x i8].
    virtual std::pair<std::vector<std::vector<uint8_t>>, std::vector<std::vector<uint8_t>>> export_raw() const = 0;
    virtual Status import_raw(const std::vector<std::vector<uint8_t>> &k_layers,
                              const std::vector<std::vector<uint8_t>> &v_layers, size_t token_count) = 0;
    virtual const GpuKvBuffer *gpu_buffer() const { return nullptr; }
    virtual const PagedKvCache *as_paged() const { return nullptr; }
};

// ---- page storage --------------------------------------------------------------

// The storage a PagePool hands out: `capacity()` pages of PAGE_SIZE rows of
// K and V; row r of page p is row id p * PAGE_SIZE + r. The library's
// implementation is DevicePageStore (a gla_pool in HBM).
class PageStore {
  public:
    virtual ~PageStore() = default;
    virtual size_t capacity() const = 0;
    virtual size_t n_kv_heads() const = 0;
    virtual size_t head_dim() const = 0;
    size_t kv_dim() const { return n_kv_heads() * head_dim(); }
    virtual gla_kv_dtype dtype() const = 0;
    // Bytes of one exported K (or V) row.
    virtual size_t row_bytes() const = 0;
    virtual Status write_rows(const int64_t *rows, size_t n, const float *k, const float *v) = 0;
    virtual Status export_rows(const int64_t *rows, size_t n, uint8_t *k, uint8_t *v) const = 0;
    virtual Status import_rows(const int64_t *rows, size_t n, const uint8_t *k, const uint8_t *v) = 0;
    virtual Status copy_page(size_t src, size_t dst) = 0;
    virtual Status zero_page(size_t page) = 0;
    // The gla_kv gla_decode / gla_prefill read, or nullptr.
    virtual const gla_kv *device_kv() const { return nullptr; }
};

class DevicePageStore final : public PageStore {
  public:
    static Result<std::shared_ptr<DevicePageStore>> create(std::shared_ptr<Device> dev, gla_kv_dtype dtype,
                                                           size_t n_kv_heads, size_t head_dim,
                                                           size_t capacity_pages);
    ~DevicePageStore() override;
    size_t capacity() const override { return capacity_; }
    size_t n_kv_heads() const override { return n_kv_heads_; }
    size_t head_dim() const override { return head_dim_; }
    gla_kv_dtype dtype() const override { return dtype_; }
    size_t row_bytes() const override;
    Status write_rows(const int64_t *rows, size_t n, const float *k, const float *v) override;
    Status export_rows(const int64_t *rows, size_t n, uint8_t *k, uint8_t *v) const override;
    Status import_rows(const int64_t *rows, size_t n, const uint8_t *k, const uint8_t *v) override;
    Status copy_page(size_t src, size_t dst) override;
    Status zero_page(size_t page) override;
    const gla_kv *device_kv() const override { return kv_; }
    const std::shared_ptr<Device> &device() const { return dev_; }

  private:
    DevicePageStore(std::shared_ptr<Device> dev, gla_kv *kv, gla_kv_dtype dtype, size_t n_kv_heads,
                    size_t head_dim, size_t capacity)
        : dev_(std::move(dev)), kv_(kv), dtype_(dtype), n_kv_heads_(n_kv_heads), head_dim_(head_dim),
          capacity_(capacity) {}
    std::shared_ptr<Device> dev_;
    gla_kv *kv_;
    gla_kv_dtype dtype_;
    size_t n_kv_heads_, head_dim_, capacity_;
};

// ---- PagePool ------------------------------------------------------------------

// src/cache/paged.rs:90-101.
struct PoolStats {
    size_t capacity = 0;   // pages the pool hands out at most
    size_t live = 0;       // pages checked out by sequences
    size_t peak_live = 0;  // high-water mark of live
    size_t pooled = 0;     // freed pages kept for reuse
    bool operator==(const PoolStats &o) const {
        return capacity == o.capacity && live == o.live && peak_live == o.peak_live && pooled == o.pooled;
    }
};

// A capacity-bounded pool of KV pages; a handle (copies share the pool), as
// src/cache/paged.rs:158-240. The store holds every page from creation (HBM
// is allocated once); pages not yet handed out count as neither live nor
// pooled, so the statistics follow the reference's lazily-allocated pool.
class PagePool {
  public:
    explicit PagePool(std::shared_ptr<PageStore> store);
    // Every page starts in the free list (src/cache/paged.rs:176-189).
    static PagePool preallocated(std::shared_ptr<PageStore> store);
    static constexpr size_t pages_for(size_t positions, size_t n_layers) {
        return (positions + PAGE_SIZE - 1) / PAGE_SIZE * n_layers;
    }
    size_t kv_dim() const;
    size_t capacity() const;
    size_t live_pages() const;
    size_t available_pages() const;
    PoolStats stats() const;
    PageStore &store() const;
    // Reference count of device page `page` (0: not handed out).
    size_t refcount(int32_t page) const;

  private:
    friend class PagedKvCache;
    struct Inner;
    std::shared_ptr<Inner> inner_;
};

// ---- PagedKvCache --------------------------------------------------------------

// Per-sequence KV cache over pages of a shared PagePool
// (src/cache/paged.rs:243-598). Move-only; pages go back to the pool on
// release() or destruction.
class PagedKvCache final : public KvStore {
  public:
    PagedKvCache(const PagePool &pool, size_t n_layers);
    ~PagedKvCache() override;
    PagedKvCache(PagedKvCache &&o) noexcept;
    PagedKvCache &operator=(PagedKvCache &&o) noexcept;
    PagedKvCache(const PagedKvCache &) = delete;
    PagedKvCache &operator=(const PagedKvCache &) = delete;

    // A new sequence sharing this one's pages for positions 0 .. upto_position
    // (paged.rs:272-310); throws Panic if upto_position > len().
    PagedKvCache fork_from(size_t upto_position) const;
    void release();
    const PagePool &pool() const { return pool_; }
    size_t n_layers() const { return table_.size(); }
    size_t pages_per_layer() const { return table_.empty() ? 0 : table_[0].size(); }
    size_t allocated_pages() const;
    size_t page_refcount(size_t layer, size_t page) const;
    bool is_page_shared(size_t layer, size_t page) const { return page_refcount(layer, page) > 1; }
    // The kv_dim-float K (V) row at pos (f32 pools: the stored floats; Q8_0
    // pools: the dequantised row).
    std::vector<float> k_at(size_t layer, size_t pos) const;
    std::vector<float> v_at(size_t layer, size_t pos) const;
    // Device page ids of `layer`, logical page i at [i] -- the page table
    // gla_decode / gla_prefill take.
    const std::vector<int32_t> &page_table(size_t layer) const { return table_.at(layer); }

    // Write n consecutive positions pos0 .. pos0+n-1 of one layer in one
    // device call (k, v: [n][kv_dim]); the chunk write of a prefill
    // (src/transformer/forward.rs:874-877). Not in the reference's API.
    void write_chunk(size_t layer, size_t pos0, size_t n, const float *k, const float *v);

    void read_k_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const override;
    void read_v_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const override;
    void write(size_t layer, size_t pos, const float *k, const float *v) override;
    Status reserve(size_t total_positions) override { return ensure_capacity(total_positions); }
    void advance() override { len_ += 1; }
    size_t len() const override { return len_; }
    void truncate(size_t new_len) override;
    std::pair<std::vector<std::vector<uint8_t>>, std::vector<std::vector<uint8_t>>> export_raw() const override;
    Status import_raw(const std::vector<std::vector<uint8_t>> &k_layers,
                      const std::vector<std::vector<uint8_t>> &v_layers, size_t token_count) override;
    const PagedKvCache *as_paged() const override { return this; }

  private:
    PagedKvCache(const PagePool &pool, std::vector<std::vector<int32_t>> table, size_t len);
    Status ensure_capacity(size_t total_positions);
    Status make_writable(size_t layer, size_t first_page, size_t last_page);
    std::vector<float> row_at(size_t layer, size_t pos, bool v) const;
    PagePool pool_;
    std::vector<std::vector<int32_t>> table_;  // table_[layer][page] = device page id
    size_t len_ = 0;
};

// ---- GpuKvCache ------------------------------------------------------------------

// Device storage of `n_seqs` contiguous caches (gla_kv_cache_create).
class GpuKvStorage;

// One sequence's device-resident contiguous cache, f32 or Q8_0: the
// GpuKvCache of src/backend/gpu.rs:1039-1104 (there f32 only, with a host
// mirror; here the rows live only in HBM and reads export them). Caches from
// one GpuBackend::create_kv_caches call share one storage, so a single
// gla_decode launch reads all of them.
class GpuKvCache final : public KvStore {
  public:
    GpuKvCache(std::shared_ptr<GpuKvStorage> storage, int seq);
    size_t kv_dim() const;
    size_t max_seq_len() const;
    gla_kv_dtype dtype() const;
    std::vector<float> k_at(size_t layer, size_t pos) const;
    std::vector<float> v_at(size_t layer, size_t pos) const;
    void write_chunk(size_t layer, size_t pos0, size_t n, const float *k, const float *v);

    void read_k_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const override;
    void read_v_head(size_t layer, size_t pos, size_t kv_h, size_t head_dim, float *buf) const override;
    void write(size_t layer, size_t pos, const float *k, const float *v) override;
    void advance() override { len_ += 1; }
    size_t len() const override { return len_; }
    void truncate(size_t new_len) override;
    std::pair<std::vector<std::vector<uint8_t>>, std::vector<std::vector<uint8_t>>> export_raw() const override;
    Status import_raw(const std::vector<std::vector<uint8_t>> &k_layers,
                      const std::vector<std::vector<uint8_t>> &v_layers, size_t token_count) override;
    const GpuKvBuffer *gpu_buffer() const override { return &buf_; }

  private:
    std::vector<float> row_at(size_t layer, size_t pos, bool v) const;
    std::shared_ptr<GpuKvStorage> storage_;
    GpuKvBuffer buf_;
    size_t len_ = 0;
};

// ---- GpuBackend --------------------------------------------------------------------

// One sequence of a batched decode step: its cache, and the window
// [window_start, window_start + attend_len) its query attends
// (src/transformer/forward.rs:574-582).
struct DecodeSeq {
    const KvStore *kv = nullptr;
    size_t window_start = 0;
    size_t attend_len = 0;
};

// One sequence of a batched prefill: its cache, its n_rows query rows and
// the absolute position of the first (src/transformer/forward.rs:879-976).
struct PrefillSeq {
    const KvStore *kv = nullptr;
    size_t n_rows = 0;
    size_t pos_offset = 0;
};

// Attention shape and numerics shared by a call.
struct AttnShape {
    uint32_t n_heads = 0;
    uint32_t n_kv_heads = 0;
    uint32_t head_dim = 0;
    float scale = 0.0f;    // query_pre_attn_scalar or 1/sqrt(head_dim)
    float softcap = 0.0f;  // attn_logit_softcapping; 0: none
};

// GGML Q8_0 weights on the device: the buffer QuantizedTensor::upload_to_gpu
// puts there (src/tensor/quantized.rs:398-401, GpuBackend::upload_buffer
// src/backend/gpu.rs:111-121), repacked once for the device matvec. Move-only;
// frees the device copy when dropped.
class GpuQ8Weights {
  public:
    GpuQ8Weights(GpuQ8Weights &&o) noexcept;
    GpuQ8Weights &operator=(GpuQ8Weights &&o) noexcept;
    GpuQ8Weights(const GpuQ8Weights &) = delete;
    GpuQ8Weights &operator=(const GpuQ8Weights &) = delete;
    ~GpuQ8Weights();
    size_t rows() const { return rows_; }
    size_t cols() const { return cols_; }
    const gla_q8w *handle() const { return w_; }

  private:
    friend class GpuBackend;
    GpuQ8Weights(std::shared_ptr<Device> dev, gla_q8w *w, size_t rows, size_t cols);
    std::shared_ptr<Device> dev_;
    gla_q8w *w_ = nullptr;
    size_t rows_ = 0, cols_ = 0;
};

class GpuBackend {
  public:
    // GpuBackend::new (src/backend/gpu.rs:44-99): GpuAdapterNotFound when no
    // device is present, which callers take as "stay on the CPU path".
    static Result<GpuBackend> create(int device = 0);
    GpuBackend(GpuBackend &&) noexcept;
    GpuBackend &operator=(GpuBackend &&) noexcept;
    ~GpuBackend();

    std::string info_string() const;
    gla_ctx *ctx() const;
    const std::shared_ptr<Device> &device() const { return dev_; }

    // src/backend/gpu.rs:266-397: q [n_heads*head_dim], k / v
    // [seq_len][n_kv_heads*head_dim] host slices -> [n_heads*head_dim]. No
    // MAX_SEQ limit; softcap applied (the shader drops it).
    Result<std::vector<float>> attention(const std::vector<float> &q, const std::vector<float> &k,
                                         const std::vector<float> &v, uint32_t n_heads, uint32_t n_kv_heads,
                                         uint32_t head_dim, uint32_t seq_len, float scale, float softcap = 0.0f);
    // src/backend/gpu.rs:860-992 over a device-resident contiguous cache.
    Result<std::vector<float>> attention_resident(const std::vector<float> &q, const GpuKvBuffer &kv_buf,
                                                  size_t layer_idx, size_t window_start, size_t attend_len,
                                                  uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                                  float scale, float softcap = 0.0f);

    // src/backend/gpu.rs:1060-1104 (f32 there; Q8_0 too here).
    Result<GpuKvCache> create_kv_cache(size_t n_layers, size_t max_seq_len, size_t n_kv_heads, size_t head_dim,
                                       gla_kv_dtype dtype = GLA_KV_F32);
    // n_seqs caches in one device storage, read together by decode_batch.
    Result<std::vector<GpuKvCache>> create_kv_caches(size_t n_seqs, size_t n_layers, size_t max_seq_len,
                                                     size_t n_kv_heads, size_t head_dim,
                                                     gla_kv_dtype dtype = GLA_KV_F32);
    // A page pool in HBM (PagePool::preallocated over a DevicePageStore).
    Result<PagePool> create_page_pool(size_t capacity_pages, size_t n_kv_heads, size_t head_dim,
                                      gla_kv_dtype dtype = GLA_KV_F32);

    // One layer's attention for a batch of single-token queries
    // (src/transformer/forward.rs:1468-1507): q [B][n_heads*head_dim] host ->
    // [B][n_heads*head_dim]. All caches must be GpuKvCaches of one storage or
    // PagedKvCaches of one device pool; otherwise GpuShaderError, and the
    // caller keeps its CPU path.
    Result<std::vector<float>> decode_batch(const std::vector<DecodeSeq> &seqs, const float *q, size_t layer,
                                            const AttnShape &shape);
    // Causal prefill of a batch of prompt chunks whose K/V are written: q
    // [sum n_rows][n_heads*head_dim] host -> same shape. sliding_window 0:
    // none. precision GLA_PREC_BF16 rounds the matrix-product inputs to bf16.
    Result<std::vector<float>> prefill_batch(const std::vector<PrefillSeq> &seqs, const float *q, size_t layer,
                                             const AttnShape &shape, size_t sliding_window = 0,
                                             gla_precision precision = GLA_PREC_F32);

    // The ops beside attention on a decode step.
    // QuantizedTensor::upload_to_gpu of a Q8_0 tensor: ggml holds rows x
    // cols/32 blocks of [f16 scale][32 x i8] (n_bytes = rows * cols / 32 * 34).
    Result<GpuQ8Weights> upload_q8_0(const uint8_t *ggml, size_t n_bytes, size_t rows, size_t cols);
    // GpuBackend::matvec_q8_0 (src/backend/gpu.rs:204-213) and
    // QuantizedTensor::matvec_batch (src/tensor/quantized.rs:302-346) in one
    // call: x [n_vec][cols] host -> [n_vec][rows].
    Result<std::vector<float>> matvec_q8_0(const GpuQ8Weights &w, const float *x, size_t n_vec);
    // tensor::rope (src/tensor/ops.rs:212-245) over n_rows rows of n_heads
    // heads, row r at position pos[r], in place on host data.
    Status rope(float *x, size_t n_rows, size_t n_heads, size_t head_dim, const int32_t *pos, float freq_base,
                float scaling_factor, size_t rot_dim);

  private:
    explicit GpuBackend(std::shared_ptr<Device> dev);
    struct Staging;
    std::shared_ptr<Device> dev_;
    std::unique_ptr<Staging> stage_;
};

// window_start of src/transformer/forward.rs:574-581.
size_t window_start(size_t pos, size_t sliding_window, bool alternating, size_t layer);

// IEEE binary16 (little-endian bytes) to f32, exact.
float f16_to_f32(uint16_t h);
// Dequantise elements [e0, e1) of a Q8_0 row (src/cache/mod.rs:318-334).
void q8_dequant_range(const uint8_t *row, size_t e0, size_t e1, float *out);

}  // namespace glint

#endif  // GLINT_HOST_HPP
