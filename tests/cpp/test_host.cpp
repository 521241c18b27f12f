// test_host.cpp -- tests of the C++ host layer (glint_amd/host/glint.hpp).
//
//   test_host            CPU: page bookkeeping over a host-memory PageStore
//                        (the cases of src/cache/paged.rs:602-1138), error
//                        types, and GpuAdapterNotFound with no device present
//   test_host --device   GPU: the same bookkeeping over the HBM page pool,
//                        then attention through GpuBackend (decode_batch,
//                        prefill_batch, attention, attention_resident) against
//                        an f64 softmax of the stored rows and the reference's
//                        bitwise invariants (paged == contiguous, fork == fresh)
//   test_host ... NAME   only the tests whose name contains NAME
//
// The bookkeeping tests keep the reference's names and assertions; their
// shape is 2 KV heads x head_dim 4 on the host store (the reference's) and
// 2 x 64 on the device (the library's smallest head_dim).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "glint.hpp"
#include "host_page_store.hpp"

using namespace glint;

namespace {

// ---- a minimal test runner ------------------------------------------------------------

struct Failure {
    std::string msg;
};

struct Case {
    const char *name;
    std::function<void()> fn;
    int where;  // 0: both modes, 1: host only, 2: device only
};

std::vector<Case> &cases() {
    static std::vector<Case> c;
    return c;
}

struct Reg {
    Reg(const char *n, std::function<void()> f, int w) { cases().push_back({n, std::move(f), w}); }
};

#define TEST_AT(name, where)                     \
    static void name();                          \
    static Reg reg_##name(#name, name, where);   \
    static void name()
#define TEST(name) TEST_AT(name, 0)
#define HOST_TEST(name) TEST_AT(name, 1)
#define DEVICE_TEST(name) TEST_AT(name, 2)

#define CHECK(cond)                                                                          \
    do {                                                                                     \
        if (!(cond)) {                                                                       \
            std::ostringstream os_;                                                          \
            os_ << __FILE__ << ":" << __LINE__ << ": CHECK(" #cond ")";                      \
            throw Failure{os_.str()};                                                        \
        }                                                                                    \
    } while (0)
#define CHECK_EQ(a, b)                                                                       \
    do {                                                                                     \
        const auto va_ = (a);                                                                \
        const auto vb_ = (b);                                                                \
        if (!(va_ == vb_)) {                                                                 \
            std::ostringstream os_;                                                          \
            os_ << __FILE__ << ":" << __LINE__ << ": " #a " == " #b " (" << va_ << " vs " << vb_ << ")"; \
            throw Failure{os_.str()};                                                        \
        }                                                                                    \
    } while (0)
#define CHECK_MSG(cond, text)                                                                \
    do {                                                                                     \
        if (!(cond)) {                                                                       \
            std::ostringstream os_;                                                          \
            os_ << __FILE__ << ":" << __LINE__ << ": " << text;                              \
            throw Failure{os_.str()};                                                        \
        }                                                                                    \
    } while (0)

// ---- the test world: host store or device pool ----------------------------------------

bool g_device = false;
std::unique_ptr<GpuBackend> g_backend;

constexpr size_t N_LAYERS = 2;
size_t N_KV_HEADS = 2;
size_t HEAD_DIM = 4;
size_t KV_DIM = 8;

GpuBackend &backend() { return *g_backend; }

// PagePool::new(capacity) of the reference: pages handed out on first use.
PagePool pool(size_t capacity_pages) {
    if (!g_device) return PagePool(std::make_shared<glint_test::HostPageStore>(capacity_pages, N_KV_HEADS, HEAD_DIM));
    auto st = DevicePageStore::create(backend().device(), GLA_KV_F32, N_KV_HEADS, HEAD_DIM, capacity_pages);
    return PagePool(std::move(st).expect("device pool"));
}

PagePool preallocated_pool(size_t capacity_pages) {
    if (!g_device)
        return PagePool::preallocated(std::make_shared<glint_test::HostPageStore>(capacity_pages, N_KV_HEADS, HEAD_DIM));
    auto st = DevicePageStore::create(backend().device(), GLA_KV_F32, N_KV_HEADS, HEAD_DIM, capacity_pages);
    return PagePool::preallocated(std::move(st).expect("device pool"));
}

// Deterministic, distinct rows (src/cache/paged.rs:617-622).
std::vector<float> row(float tag, size_t pos) {
    std::vector<float> r(KV_DIM);
    for (size_t d = 0; d < KV_DIM; d++) r[d] = tag + (float)pos * 0.25f + (float)d * 0.0625f;
    return r;
}

void append(KvStore &cache, size_t from, size_t to) {
    for (size_t pos = from; pos < to; pos++) {
        for (size_t layer = 0; layer < N_LAYERS; layer++) {
            const auto k = row((float)layer, pos);
            const auto v = row(100.0f + (float)layer, pos);
            cache.write(layer, pos, k.data(), v.data());
        }
        cache.advance();
    }
}

bool rows_equal(const std::vector<float> &a, const std::vector<float> &b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

template <class F>
std::string panic_text(F f) {
    try {
        f();
    } catch (const Panic &p) {
        return p.what();
    }
    return "";
}

// ---- equivalence with the contiguous layout ---------------------------------------------

HOST_TEST(test_paged_rows_match_formula_rows) {
    auto shared = pool(64);
    PagedKvCache paged(shared, N_LAYERS);
    append(paged, 0, 35);
    for (size_t layer = 0; layer < N_LAYERS; layer++)
        for (size_t pos = 0; pos < 35; pos++) {
            CHECK(rows_equal(paged.k_at(layer, pos), row((float)layer, pos)));
            CHECK(rows_equal(paged.v_at(layer, pos), row(100.0f + layer, pos)));
        }
}

DEVICE_TEST(test_paged_rows_match_kv_cache_rows) {
    auto plain = backend().create_kv_cache(N_LAYERS, 64, N_KV_HEADS, HEAD_DIM).expect("cache");
    PagedKvCache paged(pool(64), N_LAYERS);
    append(plain, 0, 35);
    append(paged, 0, 35);
    for (size_t layer = 0; layer < N_LAYERS; layer++)
        for (size_t pos = 0; pos < 35; pos++) {
            CHECK(rows_equal(plain.k_at(layer, pos), paged.k_at(layer, pos)));
            CHECK(rows_equal(plain.v_at(layer, pos), paged.v_at(layer, pos)));
        }
}

TEST(test_export_matches_kv_cache_bytes) {
    PagedKvCache paged(pool(64), N_LAYERS);
    append(paged, 0, 20);
    auto got = paged.export_raw();
    CHECK_EQ(got.first.size(), N_LAYERS);
    if (g_device) {
        auto plain = backend().create_kv_cache(N_LAYERS, 64, N_KV_HEADS, HEAD_DIM).expect("cache");
        append(plain, 0, 20);
        auto want = plain.export_raw();
        CHECK(want.first == got.first);
        CHECK(want.second == got.second);
    } else {  // KvCache::export_raw: native f32 bytes of rows 0 .. len
        for (size_t layer = 0; layer < N_LAYERS; layer++) {
            std::vector<uint8_t> k, v;
            for (size_t pos = 0; pos < 20; pos++) {
                auto kr = row((float)layer, pos), vr = row(100.0f + layer, pos);
                k.insert(k.end(), (uint8_t *)kr.data(), (uint8_t *)(kr.data() + KV_DIM));
                v.insert(v.end(), (uint8_t *)vr.data(), (uint8_t *)(vr.data() + KV_DIM));
            }
            CHECK(got.first[layer] == k);
            CHECK(got.second[layer] == v);
        }
    }
}

TEST(test_export_import_roundtrip) {
    auto shared = pool(64);
    PagedKvCache src(shared, N_LAYERS);
    append(src, 0, 20);
    auto kv = src.export_raw();
    PagedKvCache dst(shared, N_LAYERS);
    dst.import_raw(kv.first, kv.second, 20).expect("pool has room");
    CHECK_EQ(dst.len(), 20u);
    for (size_t layer = 0; layer < N_LAYERS; layer++)
        for (size_t pos = 0; pos < 20; pos++) {
            CHECK(rows_equal(src.k_at(layer, pos), dst.k_at(layer, pos)));
            CHECK(rows_equal(src.v_at(layer, pos), dst.v_at(layer, pos)));
        }
}

TEST(test_import_size_mismatch_is_reported) {
    PagedKvCache dst(pool(64), N_LAYERS);
    std::vector<std::vector<uint8_t>> k(N_LAYERS, std::vector<uint8_t>(20 * KV_DIM * 4)), v = k;
    v[1].resize(7);
    Status s = dst.import_raw(k, v, 20);
    CHECK(!s.ok());
    CHECK(s.error().kind() == GlintError::Kind::SnapshotCacheSizeMismatch);
    CHECK_EQ(s.error().layer(), 1u);
    CHECK_EQ(s.error().expected(), 20 * KV_DIM * 4);
    CHECK_EQ(s.error().found(), 7u);
    CHECK_EQ(s.error().to_string(),
             std::string("snapshot cache layer 1: expected ") + std::to_string(20 * KV_DIM * 4) + " bytes, found 7");
}

// ---- page accounting --------------------------------------------------------------------

TEST(test_pages_allocated_only_on_boundary_crossing) {
    auto shared = pool(64);
    PagedKvCache cache(shared, N_LAYERS);
    CHECK_EQ(shared.live_pages(), 0u);
    for (size_t pos = 0; pos < 2 * PAGE_SIZE + 1; pos++) {
        const size_t before = shared.live_pages();
        append(cache, pos, pos + 1);
        const size_t after = shared.live_pages();
        const size_t expected_new = pos % PAGE_SIZE == 0 ? N_LAYERS : 0;
        CHECK_MSG(after - before == expected_new, "pos " << pos << ": pages went " << before << " -> " << after);
    }
    CHECK_EQ(cache.pages_per_layer(), 3u);
    CHECK_EQ(shared.live_pages(), 3 * N_LAYERS);
}

TEST(test_reserve_allocates_up_front_and_write_is_free) {
    auto shared = pool(64);
    PagedKvCache cache(shared, N_LAYERS);
    cache.reserve(3 * PAGE_SIZE).expect("pool has room");
    CHECK_EQ(shared.live_pages(), 3 * N_LAYERS);
    const size_t before = shared.live_pages();
    append(cache, 0, 3 * PAGE_SIZE);
    CHECK_EQ(shared.live_pages(), before);
}

TEST(test_release_returns_pages_to_pool) {
    auto shared = pool(64);
    PagedKvCache cache(shared, N_LAYERS);
    append(cache, 0, 33);
    const size_t held = shared.live_pages();
    CHECK_EQ(held, 3 * N_LAYERS);
    cache.release();
    CHECK_EQ(shared.live_pages(), 0u);
    CHECK_EQ(shared.stats().pooled, held);
    CHECK_EQ(cache.len(), 0u);
    append(cache, 0, PAGE_SIZE);
    CHECK_EQ(shared.stats().pooled, held - N_LAYERS);
}

TEST(test_drop_returns_pages_to_pool) {
    auto shared = pool(64);
    {
        PagedKvCache cache(shared, N_LAYERS);
        append(cache, 0, 20);
        CHECK_EQ(shared.live_pages(), 2 * N_LAYERS);
    }
    CHECK_EQ(shared.live_pages(), 0u);
}

TEST(test_recycled_page_is_zeroed) {
    auto shared = pool(N_LAYERS);  // one page per layer, forces reuse
    {
        PagedKvCache first(shared, N_LAYERS);
        append(first, 0, PAGE_SIZE);
    }
    PagedKvCache second(shared, N_LAYERS);
    second.reserve(PAGE_SIZE).expect("page was returned");
    append(second, 0, 1);
    for (float x : second.k_at(0, PAGE_SIZE - 1)) CHECK_MSG(x == 0.0f, "recycled page leaked data");
    for (float x : second.v_at(1, PAGE_SIZE - 1)) CHECK_MSG(x == 0.0f, "recycled page leaked data");
}

TEST(test_truncate_keeps_pages_and_allows_rewrite) {
    auto shared = pool(64);
    PagedKvCache cache(shared, N_LAYERS);
    append(cache, 0, 33);
    const size_t held = shared.live_pages();
    cache.truncate(16);
    CHECK_EQ(cache.len(), 16u);
    CHECK_EQ(shared.live_pages(), held);
    append(cache, 16, 17);
    CHECK_EQ(shared.live_pages(), held);
    CHECK_EQ(cache.len(), 17u);
    CHECK_EQ(panic_text([&] { cache.truncate(18); }), std::string("truncate: 18 > len 17"));
}

// ---- forking, refcounts and copy-on-write ----------------------------------------------

TEST(test_fork_shares_pages_without_allocating) {
    auto shared = pool(64);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, 32);
    const size_t live_before = shared.live_pages();
    PagedKvCache child = parent.fork_from(32);
    CHECK_EQ(child.len(), 32u);
    CHECK_EQ(shared.live_pages(), live_before);
    for (size_t layer = 0; layer < N_LAYERS; layer++)
        for (size_t page = 0; page < 2; page++) {
            CHECK_EQ(parent.page_refcount(layer, page), 2u);
            CHECK(child.is_page_shared(layer, page));
        }
    for (size_t pos = 0; pos < 32; pos++) CHECK(rows_equal(parent.k_at(0, pos), child.k_at(0, pos)));
}

TEST(test_fork_drop_restores_refcount_and_frees_nothing) {
    auto shared = pool(64);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, 32);
    const size_t live = shared.live_pages();
    {
        PagedKvCache child = parent.fork_from(32);
        CHECK_EQ(child.page_refcount(0, 0), 2u);
    }
    CHECK_EQ(parent.page_refcount(0, 0), 1u);
    CHECK_EQ(shared.live_pages(), live);
}

TEST(test_fork_cow_child_write_does_not_corrupt_parent) {
    auto shared = pool(64);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, 20);
    std::vector<std::vector<float>> parent_rows;
    for (size_t p = 0; p < 20; p++) parent_rows.push_back(parent.k_at(0, p));
    PagedKvCache child = parent.fork_from(20);
    const size_t live_before = shared.live_pages();
    CHECK(child.is_page_shared(0, 1));
    for (size_t layer = 0; layer < N_LAYERS; layer++) {
        const auto k = row(7.0f, 20), v = row(8.0f, 20);
        child.write(layer, 20, k.data(), v.data());
    }
    child.advance();
    CHECK_EQ(shared.live_pages(), live_before + N_LAYERS);
    CHECK(!child.is_page_shared(0, 1));
    CHECK(!parent.is_page_shared(0, 1));
    CHECK_EQ(parent.page_refcount(0, 0), 2u);
    CHECK_EQ(parent.len(), 20u);
    for (size_t pos = 0; pos < 20; pos++) CHECK(rows_equal(parent.k_at(0, pos), parent_rows[pos]));
    for (size_t pos = 0; pos < 20; pos++) CHECK(rows_equal(child.k_at(0, pos), parent_rows[pos]));
    CHECK(rows_equal(child.k_at(0, 20), row(7.0f, 20)));
}

TEST(test_fork_cow_parent_write_does_not_corrupt_child) {
    auto shared = pool(64);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, 20);
    PagedKvCache child = parent.fork_from(20);
    std::vector<std::vector<float>> child_rows;
    for (size_t p = 0; p < 20; p++) child_rows.push_back(child.k_at(0, p));
    append(parent, 20, 24);
    CHECK(!parent.is_page_shared(0, 1));
    for (size_t pos = 0; pos < 20; pos++) CHECK(rows_equal(child.k_at(0, pos), child_rows[pos]));
    CHECK_EQ(child.len(), 20u);
}

TEST(test_fork_on_page_boundary_needs_no_copy) {
    auto shared = pool(64);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, PAGE_SIZE);
    PagedKvCache child = parent.fork_from(PAGE_SIZE);
    CHECK_EQ(child.pages_per_layer(), 1u);
    const size_t live_before = shared.live_pages();
    append(child, PAGE_SIZE, PAGE_SIZE + 1);
    CHECK_EQ(shared.live_pages(), live_before + N_LAYERS);
    CHECK(child.is_page_shared(0, 0));
}

TEST(test_fork_partial_prefix) {
    auto shared = pool(64);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, 40);
    PagedKvCache child = parent.fork_from(18);
    CHECK_EQ(child.len(), 18u);
    CHECK_EQ(child.pages_per_layer(), 2u);
    for (size_t pos = 0; pos < 18; pos++) CHECK(rows_equal(child.k_at(0, pos), parent.k_at(0, pos)));
    CHECK_EQ(parent.page_refcount(0, 2), 1u);
}

TEST(test_fork_beyond_len_panics) {
    auto shared = pool(64);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, 4);
    const std::string text = panic_text([&] { (void)parent.fork_from(5); });
    CHECK_MSG(text.find("fork_from") != std::string::npos, "no fork_from panic: '" << text << "'");
}

// ---- pool exhaustion ---------------------------------------------------------------------

TEST(test_pool_exhaustion_is_recoverable) {
    auto shared = pool(2 * N_LAYERS);
    auto first = std::make_unique<PagedKvCache>(shared, N_LAYERS);
    append(*first, 0, PAGE_SIZE);
    PagedKvCache second(shared, N_LAYERS);
    append(second, 0, PAGE_SIZE);
    CHECK_EQ(shared.available_pages(), 0u);
    Status err = second.reserve(PAGE_SIZE + 1);
    CHECK(!err.ok());
    CHECK(err.error().kind() == GlintError::Kind::KvPagePoolExhausted);
    CHECK_EQ(first->len(), PAGE_SIZE);
    CHECK_EQ(second.len(), PAGE_SIZE);
    for (size_t pos = 0; pos < PAGE_SIZE; pos++) {
        CHECK(rows_equal(first->k_at(0, pos), row(0.0f, pos)));
        CHECK(rows_equal(second.k_at(1, pos), row(1.0f, pos)));
    }
    CHECK_EQ(shared.live_pages(), 2 * N_LAYERS);
    first.reset();
    second.reserve(PAGE_SIZE + 1).expect("pages were returned");
    append(second, PAGE_SIZE, PAGE_SIZE + 1);
    CHECK_EQ(second.len(), PAGE_SIZE + 1);
}

TEST(test_exhausted_reserve_reports_the_shortfall) {
    auto shared = pool(N_LAYERS);
    PagedKvCache cache(shared, N_LAYERS);
    cache.reserve(PAGE_SIZE).expect("first page fits");
    Status s = cache.reserve(4 * PAGE_SIZE);
    CHECK(!s.ok());
    CHECK(s.error().kind() == GlintError::Kind::KvPagePoolExhausted);
    CHECK_EQ(s.error().needed(), 3 * N_LAYERS);
    CHECK_EQ(s.error().available(), 0u);
    CHECK_EQ(s.error().capacity(), N_LAYERS);
    CHECK_EQ(s.error().to_string(), std::string("KV page pool exhausted: needed 6 page(s), 0 of 2 free"));
}

TEST(test_cow_reports_exhaustion_instead_of_sharing) {
    auto shared = pool(N_LAYERS);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, 4);
    PagedKvCache child = parent.fork_from(4);
    CHECK_EQ(shared.available_pages(), 0u);
    Status err = child.reserve(5);
    CHECK(!err.ok());
    CHECK(err.error().kind() == GlintError::Kind::KvPagePoolExhausted);
    CHECK(child.is_page_shared(0, 0));
    CHECK(rows_equal(parent.k_at(0, 3), row(0.0f, 3)));
}

TEST(test_write_without_reserve_panics_when_exhausted) {
    auto shared = pool(N_LAYERS);
    PagedKvCache cache(shared, N_LAYERS);
    append(cache, 0, PAGE_SIZE);
    const std::string text = panic_text([&] { append(cache, PAGE_SIZE, PAGE_SIZE + 1); });
    CHECK_MSG(text.find("call KvStore::reserve()") != std::string::npos, "panic text: '" << text << "'");
}

// ---- pool bookkeeping --------------------------------------------------------------------

TEST(test_pages_for_and_stats) {
    CHECK_EQ(PagePool::pages_for(0, 4), 0u);
    CHECK_EQ(PagePool::pages_for(1, 4), 4u);
    CHECK_EQ(PagePool::pages_for(PAGE_SIZE, 4), 4u);
    CHECK_EQ(PagePool::pages_for(PAGE_SIZE + 1, 4), 8u);
    auto shared = pool(10);
    CHECK_EQ(shared.kv_dim(), KV_DIM);
    CHECK_EQ(shared.capacity(), 10u);
    {
        PagedKvCache cache(shared, N_LAYERS);
        append(cache, 0, PAGE_SIZE + 1);
        CHECK_EQ(cache.allocated_pages(), 2 * N_LAYERS);
    }
    const PoolStats stats = shared.stats();
    CHECK_EQ(stats.capacity, 10u);
    CHECK_EQ(stats.live, 0u);
    CHECK_EQ(stats.peak_live, 2 * N_LAYERS);
    CHECK_EQ(stats.pooled, 2 * N_LAYERS);
}

TEST(test_preallocated_pool_hands_out_ready_buffers) {
    auto shared = preallocated_pool(4);
    CHECK_EQ(shared.stats().pooled, 4u);
    PagedKvCache cache(shared, N_LAYERS);
    append(cache, 0, 1);
    CHECK_EQ(shared.stats().pooled, 4 - N_LAYERS);
    CHECK_EQ(shared.live_pages(), N_LAYERS);
}

HOST_TEST(test_copy_on_write_copies_and_recycling_wipes) {
    auto store = std::make_shared<glint_test::HostPageStore>(8, N_KV_HEADS, HEAD_DIM);
    PagePool shared(store);
    {
        PagedKvCache parent(shared, 1);
        const auto k = row(1.0f, 0);
        parent.write(0, 0, k.data(), k.data());
        parent.advance();
        PagedKvCache child = parent.fork_from(1);
        child.write(0, 1, k.data(), k.data());  // tail page shared: one copy
        CHECK_EQ(store->copies, 1u);
        CHECK_EQ(store->wipes, 0u);  // fresh pages are zero from creation
    }
    PagedKvCache again(shared, 1);
    again.reserve(1).expect("room");
    CHECK_EQ(store->wipes, 1u);  // a returned page is wiped before reuse
}

HOST_TEST(test_no_device_reports_adapter_not_found) {
    Result<GpuBackend> be = GpuBackend::create(0);
    if (be.ok()) return;  // a device is present: nothing to check here
    CHECK(be.error().kind() == GlintError::Kind::GpuAdapterNotFound);
}

// Seeded N(0,1) values (xorshift64 + Box-Muller).
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed ? seed : 1) {}
    double uniform() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return ((double)(s >> 40) + 0.5) / 16777216.0;
    }
    std::vector<float> normal(size_t n, double mul = 1.0) {
        std::vector<float> v(n);
        for (size_t i = 0; i < n; i += 2) {
            const double r = std::sqrt(-2.0 * std::log(uniform())), t = 6.283185307179586 * uniform();
            v[i] = (float)(r * std::cos(t) * mul);
            if (i + 1 < n) v[i + 1] = (float)(r * std::sin(t) * mul);
        }
        return v;
    }
};

// ---- page-sharing fork over a device pool -------------------------------------------------

// A cache holding tokens.size() positions, rows derived from the token ids.
PagedKvCache filled(const PagePool &shared, const std::vector<uint32_t> &tokens) {
    PagedKvCache cache(shared, N_LAYERS);
    cache.reserve(tokens.size()).expect("pool has room");
    for (size_t pos = 0; pos < tokens.size(); pos++) {
        for (size_t layer = 0; layer < N_LAYERS; layer++) {
            std::vector<float> k(KV_DIM), v(KV_DIM);
            for (size_t d = 0; d < KV_DIM; d++) {
                k[d] = (float)tokens[pos] + (float)layer * 0.5f + (float)d * 0.125f;
                v[d] = k[d] + 100.0f;
            }
            cache.write(layer, pos, k.data(), v.data());
        }
        cache.advance();
    }
    return cache;
}

std::vector<uint32_t> prompt(size_t len, uint32_t tag) {
    std::vector<uint32_t> t(len);
    for (size_t i = 0; i < len; i++) t[i] = (uint32_t)i * 7 + tag;
    return t;
}

std::vector<uint32_t> cat(std::vector<uint32_t> a, const std::vector<uint32_t> &b) {
    a.insert(a.end(), b.begin(), b.end());
    return a;
}

// A sequence forked from another's whole-page prefix (the pages an engine-side
// prefix registry hands out, src/cache/paged.rs:433-444) and then given its
// own suffix decodes bit for bit like a sequence that computed the whole
// prompt itself (device). The suffix's first write copies the shared partial
// page on write.
DEVICE_TEST(test_fork_decode_equals_cold_sequence) {
    auto shared = pool(256);
    auto base = prompt(70, 0);
    PagedKvCache parent = filled(shared, base);
    PagedKvCache fork = parent.fork_from(64);
    CHECK_EQ(fork.len(), 64u);
    auto full = cat(base, prompt(25, 3));
    fork.reserve(full.size()).expect("room");
    for (size_t pos = 64; pos < full.size(); pos++) {
        for (size_t layer = 0; layer < N_LAYERS; layer++) {
            std::vector<float> k(KV_DIM), v(KV_DIM);
            for (size_t d = 0; d < KV_DIM; d++) {
                k[d] = (float)full[pos] + (float)layer * 0.5f + (float)d * 0.125f;
                v[d] = k[d] + 100.0f;
            }
            fork.write(layer, pos, k.data(), v.data());
        }
        fork.advance();
    }
    PagedKvCache cold = filled(shared, full);
    const AttnShape shape{(uint32_t)(2 * N_KV_HEADS), (uint32_t)N_KV_HEADS, (uint32_t)HEAD_DIM, 0.05f, 0.0f};
    Rng rng(91);
    const auto q = rng.normal(2 * N_KV_HEADS * HEAD_DIM);
    for (size_t layer = 0; layer < N_LAYERS; layer++) {
        auto a = backend().decode_batch({{&fork, 0, full.size()}}, q.data(), layer, shape).expect("fork");
        auto b = backend().decode_batch({{&cold, 0, full.size()}}, q.data(), layer, shape).expect("cold");
        CHECK(rows_equal(a, b));
    }
}

// ---- attention through GpuBackend (device) -------------------------------------------------

// f64 softmax attention of one q head over rows [start, start + n) read back
// from the cache (the stored values: dequantised for Q8_0).
std::vector<double> attend_f64(const float *q, const std::vector<std::vector<float>> &K,
                               const std::vector<std::vector<float>> &V, size_t kv_h, size_t d, double scale,
                               double softcap) {
    std::vector<double> out(d, 0.0);
    if (K.empty()) return out;
    std::vector<double> s(K.size());
    double m = -INFINITY;
    for (size_t j = 0; j < K.size(); j++) {
        double acc = 0.0;
        for (size_t i = 0; i < d; i++) acc += (double)q[i] * K[j][kv_h * d + i];
        acc *= scale;
        if (softcap > 0.0) acc = softcap * std::tanh(acc / softcap);
        s[j] = acc;
        m = std::max(m, acc);
    }
    double l = 0.0;
    for (size_t j = 0; j < K.size(); j++) {
        s[j] = std::exp(s[j] - m);
        l += s[j];
    }
    for (size_t j = 0; j < K.size(); j++)
        for (size_t i = 0; i < d; i++) out[i] += s[j] / l * V[j][kv_h * d + i];
    return out;
}

void check_close(const float *got, const std::vector<double> &want, const std::string &what) {
    for (size_t i = 0; i < want.size(); i++) {
        const double err = std::fabs((double)got[i] - want[i]);
        CHECK_MSG(std::isfinite(got[i]) && (err <= 1e-4 || err <= 1e-3 * std::fabs(want[i])),
                  what << " [" << i << "]: got " << got[i] << " want " << want[i]);
    }
}


// Decode over paged and contiguous caches of one shape, f32 and Q8_0, with
// GQA, ragged lengths, windows starting mid-page and a soft-cap, against the
// f64 softmax of the rows the caches hold.
DEVICE_TEST(test_decode_batch_matches_f64) {
    struct Shape {
        uint32_t H, Hkv, d;
        float softcap;
    };
    const Shape shapes[] = {{8, 2, 64, 0.0f}, {8, 2, 128, 30.0f}, {4, 2, 256, 50.0f}};
    const size_t lens[] = {1, 17, 100, 203};
    for (const Shape &sh : shapes)
        for (gla_kv_dtype dt : {GLA_KV_F32, GLA_KV_Q8_0}) {
            const size_t kv_dim = (size_t)sh.Hkv * sh.d, B = 4, layers = 2, max_seq = 208;
            auto pool_r = backend().create_page_pool(B * layers * (max_seq / PAGE_SIZE), sh.Hkv, sh.d, dt);
            PagePool shared = std::move(pool_r).expect("pool");
            auto contig = backend().create_kv_caches(B, layers, max_seq, sh.Hkv, sh.d, dt).expect("caches");
            std::vector<PagedKvCache> paged;
            Rng rng(0x5eed + sh.d + dt);
            for (size_t b = 0; b < B; b++) {
                paged.emplace_back(shared, layers);
                paged[b].reserve(lens[b]).expect("room");
                for (size_t l = 0; l < layers; l++) {
                    const auto k = rng.normal(lens[b] * kv_dim), v = rng.normal(lens[b] * kv_dim);
                    paged[b].write_chunk(l, 0, lens[b], k.data(), v.data());
                    contig[b].write_chunk(l, 0, lens[b], k.data(), v.data());
                }
            }
            const AttnShape shape{sh.H, sh.Hkv, sh.d, 1.0f / std::sqrt((float)sh.d), sh.softcap};
            const auto q = rng.normal(B * sh.H * sh.d);
            for (size_t layer = 0; layer < layers; layer++) {
                std::vector<DecodeSeq> ps, cs;
                for (size_t b = 0; b < B; b++) {
                    const size_t ws = window_start(lens[b] - 1, 37, false, layer);  // window 37
                    ps.push_back({&paged[b], ws, lens[b] - ws});
                    cs.push_back({&contig[b], ws, lens[b] - ws});
                }
                const auto got_p = backend().decode_batch(ps, q.data(), layer, shape).expect("paged decode");
                const auto got_c = backend().decode_batch(cs, q.data(), layer, shape).expect("contig decode");
                for (size_t b = 0; b < B; b++) {
                    std::vector<std::vector<float>> K, V;
                    for (size_t p = ps[b].window_start; p < lens[b]; p++) {
                        K.push_back(paged[b].k_at(layer, p));
                        V.push_back(paged[b].v_at(layer, p));
                    }
                    for (uint32_t h = 0; h < sh.H; h++) {
                        const size_t o = (b * sh.H + h) * sh.d;
                        const auto want = attend_f64(&q[o], K, V, h / (sh.H / sh.Hkv), sh.d, shape.scale, sh.softcap);
                        std::ostringstream w;
                        w << "d" << sh.d << (dt == GLA_KV_Q8_0 ? " q8" : " f32") << " layer " << layer << " seq " << b
                          << " head " << h;
                        check_close(&got_p[o], want, w.str() + " paged");
                        check_close(&got_c[o], want, w.str() + " contiguous");
                    }
                }
            }
        }
}

// src/cache/paged.rs:655-707 through the GPU: the paged cache and the
// contiguous cache give bit-identical attention, also for a window that
// starts and ends mid-page (13, 21).
DEVICE_TEST(test_paged_flash_output_matches_kv_cache_bitwise) {
    auto plain = backend().create_kv_cache(N_LAYERS, 64, N_KV_HEADS, HEAD_DIM).expect("cache");
    PagedKvCache paged(pool(64), N_LAYERS);
    append(plain, 0, 37);
    append(paged, 0, 37);
    CHECK_EQ(plain.len(), paged.len());
    const AttnShape shape{(uint32_t)N_KV_HEADS, (uint32_t)N_KV_HEADS, (uint32_t)HEAD_DIM,
                          1.0f / std::sqrt((float)HEAD_DIM), 0.0f};
    std::vector<float> q(N_KV_HEADS * HEAD_DIM);
    for (size_t d = 0; d < q.size(); d++) q[d] = (float)(d % HEAD_DIM) * 0.3f - 0.4f;
    for (size_t layer = 0; layer < N_LAYERS; layer++)
        for (auto win : {std::pair<size_t, size_t>{0, 37}, {13, 21}}) {
            auto want = backend().decode_batch({{&plain, win.first, win.second}}, q.data(), layer, shape).expect("d");
            auto got = backend().decode_batch({{&paged, win.first, win.second}}, q.data(), layer, shape).expect("d");
            CHECK(rows_equal(want, got));
        }
}

// A forked sequence attends exactly like a fresh one holding the same rows
// (src/transformer/forward.rs:1851-1886), after copy-on-write of its tail.
DEVICE_TEST(test_fork_decode_equals_fresh) {
    auto shared = pool(64);
    PagedKvCache parent(shared, N_LAYERS);
    append(parent, 0, 40);
    PagedKvCache child = parent.fork_from(21);
    PagedKvCache fresh(shared, N_LAYERS);
    append(fresh, 0, 21);
    for (size_t pos = 21; pos < 30; pos++) {
        for (size_t layer = 0; layer < N_LAYERS; layer++) {
            const auto k = row(50.0f + layer, pos), v = row(60.0f + layer, pos);
            child.write(layer, pos, k.data(), v.data());
            fresh.write(layer, pos, k.data(), v.data());
        }
        child.advance();
        fresh.advance();
    }
    const AttnShape shape{(uint32_t)(2 * N_KV_HEADS), (uint32_t)N_KV_HEADS, (uint32_t)HEAD_DIM, 0.125f, 0.0f};
    Rng rng(77);
    const auto q = rng.normal(2 * N_KV_HEADS * HEAD_DIM);
    for (size_t layer = 0; layer < N_LAYERS; layer++) {
        auto a = backend().decode_batch({{&child, 0, 30}}, q.data(), layer, shape).expect("child");
        auto b = backend().decode_batch({{&fresh, 0, 30}}, q.data(), layer, shape).expect("fresh");
        CHECK(rows_equal(a, b));
        // the parent still attends its own rows 21..39
        auto c = backend().decode_batch({{&parent, 0, 30}}, q.data(), layer, shape).expect("parent");
        CHECK(!rows_equal(a, c));
    }
}

// Causal prefill of two prompt chunks (one at an offset) on a paged Q8_0
// cache and a contiguous f32 cache, sliding window 9, against f64.
DEVICE_TEST(test_prefill_batch_matches_f64) {
    const uint32_t H = 4, Hkv = 2, d = 128;
    const size_t kv_dim = (size_t)Hkv * d;
    const size_t n_rows[] = {33, 20}, offs[] = {0, 11};
    for (gla_kv_dtype dt : {GLA_KV_F32, GLA_KV_Q8_0}) {
        PagePool shared = backend().create_page_pool(16, Hkv, d, dt).expect("pool");
        std::vector<PagedKvCache> seqs;
        Rng rng(900 + dt);
        for (size_t b = 0; b < 2; b++) {
            seqs.emplace_back(shared, 1);
            const size_t n = offs[b] + n_rows[b];
            seqs[b].reserve(n).expect("room");
            const auto k = rng.normal(n * kv_dim), v = rng.normal(n * kv_dim);
            seqs[b].write_chunk(0, 0, n, k.data(), v.data());
        }
        const AttnShape shape{H, Hkv, d, 1.0f / std::sqrt((float)d), 0.0f};
        const auto q = rng.normal((n_rows[0] + n_rows[1]) * H * d);
        std::vector<PrefillSeq> ps = {{&seqs[0], n_rows[0], offs[0]}, {&seqs[1], n_rows[1], offs[1]}};
        const auto got = backend().prefill_batch(ps, q.data(), 0, shape, 9).expect("prefill");
        size_t r0 = 0;
        for (size_t b = 0; b < 2; b++) {
            for (size_t r = 0; r < n_rows[b]; r++) {
                const size_t pos = offs[b] + r, w = pos + 1 > 9 ? pos + 1 - 9 : 0;
                std::vector<std::vector<float>> K, V;
                for (size_t p = w; p <= pos; p++) {
                    K.push_back(seqs[b].k_at(0, p));
                    V.push_back(seqs[b].v_at(0, p));
                }
                for (uint32_t h = 0; h < H; h++) {
                    const size_t o = ((r0 + r) * H + h) * d;
                    check_close(&got[o], attend_f64(&q[o], K, V, h / (H / Hkv), d, shape.scale, 0.0),
                                "prefill seq " + std::to_string(b) + " row " + std::to_string(r));
                }
            }
            r0 += n_rows[b];
        }
    }
}

// GpuBackend::attention / attention_resident (src/backend/gpu.rs:266, :860).
DEVICE_TEST(test_attention_and_resident_match_f64) {
    const uint32_t H = 8, Hkv = 2, d = 64, S = 300;
    const size_t kv_dim = (size_t)Hkv * d;
    Rng rng(31);
    const auto q = rng.normal(H * d), k = rng.normal(S * kv_dim), v = rng.normal(S * kv_dim);
    const float scale = 0.125f;
    auto got = backend().attention(q, k, v, H, Hkv, d, S, scale, 20.0f).expect("attention");
    std::vector<std::vector<float>> K(S), V(S);
    for (size_t j = 0; j < S; j++) {
        K[j].assign(k.begin() + (ptrdiff_t)(j * kv_dim), k.begin() + (ptrdiff_t)((j + 1) * kv_dim));
        V[j].assign(v.begin() + (ptrdiff_t)(j * kv_dim), v.begin() + (ptrdiff_t)((j + 1) * kv_dim));
    }
    for (uint32_t h = 0; h < H; h++)
        check_close(&got[h * d], attend_f64(&q[h * d], K, V, h / (H / Hkv), d, scale, 20.0), "attention");

    auto cache = backend().create_kv_cache(1, 512, Hkv, d).expect("cache");
    cache.write_chunk(0, 0, S, k.data(), v.data());
    for (size_t s = 0; s < S; s++) cache.advance();
    const size_t ws = 100, n = 150;
    auto res = backend()
                   .attention_resident(q, *cache.gpu_buffer(), 0, ws, n, H, Hkv, d, scale)
                   .expect("attention_resident");
    std::vector<std::vector<float>> Kw(K.begin() + ws, K.begin() + ws + n), Vw(V.begin() + ws, V.begin() + ws + n);
    for (uint32_t h = 0; h < H; h++)
        check_close(&res[h * d], attend_f64(&q[h * d], Kw, Vw, h / (H / Hkv), d, scale, 0.0), "resident");
    Result<std::vector<float>> bad = backend().attention_resident(q, *cache.gpu_buffer(), 0, 0, 10, H, Hkv, 128, scale);
    CHECK(!bad.ok() && bad.error().kind() == GlintError::Kind::GpuShaderError);
}

// Paged Q8_0 rows are the KvCacheQ8 rows, byte for byte (the composition
// the reference has no type for).
DEVICE_TEST(test_q8_paged_rows_equal_contiguous_rows) {
    PagePool shared = backend().create_page_pool(8, 2, 64, GLA_KV_Q8_0).expect("pool");
    PagedKvCache paged(shared, 1);
    auto contig = backend().create_kv_cache(1, 64, 2, 64, GLA_KV_Q8_0).expect("cache");
    Rng rng(5);
    const auto k = rng.normal(40 * 128, 3.0), v = rng.normal(40 * 128);
    paged.reserve(40).expect("room");
    paged.write_chunk(0, 0, 40, k.data(), v.data());
    contig.write_chunk(0, 0, 40, k.data(), v.data());
    for (size_t i = 0; i < 40; i++) {
        paged.advance();
        contig.advance();
    }
    CHECK(paged.export_raw() == contig.export_raw());
    std::vector<float> a(64), b(64);
    paged.read_v_head(0, 39, 1, 64, a.data());
    contig.read_v_head(0, 39, 1, 64, b.data());
    CHECK(rows_equal(a, b));
}

DEVICE_TEST(test_mixed_caches_are_rejected) {
    auto plain = backend().create_kv_cache(N_LAYERS, 64, N_KV_HEADS, HEAD_DIM).expect("cache");
    PagedKvCache paged(pool(64), N_LAYERS);
    append(plain, 0, 5);
    append(paged, 0, 5);
    const AttnShape shape{(uint32_t)N_KV_HEADS, (uint32_t)N_KV_HEADS, (uint32_t)HEAD_DIM, 0.1f, 0.0f};
    std::vector<float> q(2 * N_KV_HEADS * HEAD_DIM, 0.5f);
    auto r = backend().decode_batch({{&plain, 0, 5}, {&paged, 0, 5}}, q.data(), 0, shape);
    CHECK(!r.ok() && r.error().kind() == GlintError::Kind::GpuShaderError);
    auto over = backend().decode_batch({{&paged, 0, 17}}, q.data(), 0, shape);  // past the held pages
    CHECK(!over.ok() && over.error().kind() == GlintError::Kind::GpuShaderError);
}

DEVICE_TEST(test_fixed_caches_reserve_is_a_noop) {
    auto plain = backend().create_kv_cache(1, 8, 1, 64).expect("cache");
    CHECK(plain.reserve(1000000).ok());
}

// ---- the ops beside attention (src/tensor/quantized.rs, src/tensor/ops.rs) -----------------

// One GGML Q8_0 block: [f16 scale LE][32 x i8].
void push_block(std::vector<uint8_t> &out, uint16_t scale_bits, const int8_t *q) {
    out.push_back((uint8_t)(scale_bits & 0xff));
    out.push_back((uint8_t)(scale_bits >> 8));
    for (int j = 0; j < 32; j++) out.push_back((uint8_t)q[j]);
}

// quantized.rs test_q8_0_matvec_matches_f32: rows [0..31] x scale 1.0 and
// [0, -1, .., -31] x scale 2.0 against [0..31] give 10416 and -20832 (exact:
// integer products and sums below 2^24).
DEVICE_TEST(test_matvec_q8_0_reference_fixture) {
    std::vector<uint8_t> raw;
    int8_t a[32], b[32];
    for (int j = 0; j < 32; j++) a[j] = (int8_t)j, b[j] = (int8_t)-j;
    push_block(raw, 0x3C00, a);  // 1.0
    push_block(raw, 0x4000, b);  // 2.0
    auto w = backend().upload_q8_0(raw.data(), raw.size(), 2, 32).expect("upload");
    CHECK_EQ(w.rows(), 2u);
    CHECK_EQ(w.cols(), 32u);
    std::vector<float> x(32);
    for (int j = 0; j < 32; j++) x[j] = (float)j;
    const auto y = backend().matvec_q8_0(w, x.data(), 1).expect("matvec");
    CHECK_EQ(y.size(), 2u);
    CHECK_EQ(y[0], 10416.0f);
    CHECK_EQ(y[1], -20832.0f);
}

// Random Q8_0 matrices (row tails, odd block counts, the vector-ALU and the
// MFMA paths) against the f64 product of the dequantised rows: within 2e-6
// of sum |x * w| per output.
DEVICE_TEST(test_matvec_q8_0_matches_f64) {
    struct Shape {
        size_t rows, cols, n_vec;
    };
    const Shape shapes[] = {{100, 96, 3}, {64, 4096, 1}, {48, 512, 20}, {16, 32, 70}};
    Rng rng(0x0a7e);
    for (const Shape &sh : shapes) {
        const size_t nb = sh.cols / 32;
        std::vector<uint8_t> raw;
        std::vector<double> wd(sh.rows * sh.cols);
        for (size_t r = 0; r < sh.rows; r++)
            for (size_t blk = 0; blk < nb; blk++) {
                int8_t q[32];
                for (int j = 0; j < 32; j++) q[j] = (int8_t)((int)(rng.uniform() * 255.0) - 127);
                // a normal f16 in [2^-12, 2^-2): exponent field 3..12, random mantissa
                const uint16_t bits = (uint16_t)(((3 + (int)(rng.uniform() * 10.0)) << 10) | (int)(rng.uniform() * 1024.0));
                push_block(raw, bits, q);
                const double sc = f16_to_f32(bits);
                for (int j = 0; j < 32; j++) wd[r * sh.cols + blk * 32 + j] = sc * q[j];
            }
        auto w = backend().upload_q8_0(raw.data(), raw.size(), sh.rows, sh.cols).expect("upload");
        const auto x = rng.normal(sh.n_vec * sh.cols);
        const auto y = backend().matvec_q8_0(w, x.data(), sh.n_vec).expect("matvec");
        CHECK_EQ(y.size(), sh.n_vec * sh.rows);
        for (size_t v = 0; v < sh.n_vec; v++)
            for (size_t r = 0; r < sh.rows; r++) {
                double exact = 0.0, mag = 0.0;
                for (size_t c = 0; c < sh.cols; c++) {
                    exact += (double)x[v * sh.cols + c] * wd[r * sh.cols + c];
                    mag += std::fabs((double)x[v * sh.cols + c] * wd[r * sh.cols + c]);
                }
                CHECK_MSG(std::fabs(y[v * sh.rows + r] - exact) <= 2e-6 * mag,
                          sh.rows << "x" << sh.cols << " vec " << v << " row " << r << ": " << y[v * sh.rows + r]
                                  << " vs " << exact);
            }
    }
}

DEVICE_TEST(test_upload_q8_0_rejects_bad_sizes) {
    std::vector<uint8_t> raw(34 * 4, 0);
    CHECK(!backend().upload_q8_0(raw.data(), raw.size(), 2, 48).ok());      // cols not a multiple of 32
    CHECK(!backend().upload_q8_0(raw.data(), raw.size() - 1, 2, 64).ok());  // short buffer
    auto w = backend().upload_q8_0(raw.data(), raw.size(), 2, 64).expect("upload");
    auto moved = std::move(w);
    CHECK(moved.handle() != nullptr);
    CHECK(w.handle() == nullptr);
}

// ops.rs tests through the host layer: position 0 is the identity (full and
// partial rotary); pos 2 at scaling 2 equals pos 1 at scaling 1 bit for bit;
// dimensions past rot_dim (and an odd head_dim's last one) are untouched; and
// the rotation against the f64 one, within the f32 angle's own rounding.
DEVICE_TEST(test_rope_through_host_layer) {
    {
        std::vector<float> x = {1.0f, 2.0f, 3.0f, 4.0f};
        const int32_t p0 = 0;
        for (size_t rot : {4, 2}) {
            std::vector<float> y = x;
            backend().rope(y.data(), 1, 1, 4, &p0, 10000.0f, 1.0f, rot).expect("rope");
            CHECK(y == x);
        }
        std::vector<float> a = x, b = x;
        const int32_t p2 = 2, p1 = 1;
        backend().rope(a.data(), 1, 1, 4, &p2, 10000.0f, 2.0f, 4).expect("rope");
        backend().rope(b.data(), 1, 1, 4, &p1, 10000.0f, 1.0f, 4).expect("rope");
        CHECK(a == b);
    }
    const size_t heads = 3;
    const int32_t pos[] = {0, 1, 17, 4095, 65535};
    const size_t n_rows = sizeof(pos) / sizeof(pos[0]);
    struct Case {
        size_t head_dim, rot_dim;
        float base, scaling;
    };
    const Case cases_[] = {{8, 8, 10000.0f, 1.0f}, {8, 6, 500000.0f, 2.0f}, {5, 5, 10000.0f, 1.0f}};
    Rng rng(0x20be);
    for (const Case &c : cases_) {
        const auto x = rng.normal(n_rows * heads * c.head_dim);
        std::vector<float> y = x;
        backend().rope(y.data(), n_rows, heads, c.head_dim, pos, c.base, c.scaling, c.rot_dim).expect("rope");
        const size_t rot = std::min(c.rot_dim, c.head_dim) & ~(size_t)1;
        for (size_t r = 0; r < n_rows; r++)
            for (size_t h = 0; h < heads; h++) {
                const size_t o = (r * heads + h) * c.head_dim;
                for (size_t i = rot; i < c.head_dim; i++) CHECK(y[o + i] == x[o + i]);
                const double ps = (double)pos[r] / c.scaling;
                for (size_t i = 0; i < rot; i += 2) {
                    const double ang = ps * std::pow((double)c.base, -(double)i / (double)c.head_dim);
                    const double w0 = x[o + i] * std::cos(ang) - x[o + i + 1] * std::sin(ang);
                    const double w1 = x[o + i] * std::sin(ang) + x[o + i + 1] * std::cos(ang);
                    // f32 angles carry up to ~ps * 2^-23 rad of rounding
                    const double tol = (2e-6 + ps * 2.4e-7) * (std::fabs(x[o + i]) + std::fabs(x[o + i + 1]));
                    CHECK_MSG(std::fabs(y[o + i] - w0) <= tol && std::fabs(y[o + i + 1] - w1) <= tol,
                              "hd " << c.head_dim << " pos " << pos[r] << " i " << i << ": " << y[o + i] << ","
                                    << y[o + i + 1] << " vs " << w0 << "," << w1);
                }
            }
    }
}

}  // namespace

int main(int argc, char **argv) {
    std::string filter;
    for (int i = 1; i < argc; i++) {
        if (std::strcmp(argv[i], "--device") == 0)
            g_device = true;
        else
            filter = argv[i];
    }
    if (g_device) {
        Result<GpuBackend> be = GpuBackend::create(0);
        if (!be.ok()) {
            std::printf("no device: %s\n", be.error().to_string().c_str());
            return 2;
        }
        g_backend = std::make_unique<GpuBackend>(std::move(be).value());
        N_KV_HEADS = 2;
        HEAD_DIM = 64;
        KV_DIM = N_KV_HEADS * HEAD_DIM;
        std::printf("device: %s\n", g_backend->info_string().c_str());
    }
    int run = 0, failed = 0;
    for (const Case &c : cases()) {
        if (c.where == (g_device ? 1 : 2)) continue;
        if (!filter.empty() && std::string(c.name).find(filter) == std::string::npos) continue;
        run++;
        std::printf("%-60s ", c.name);
        std::fflush(stdout);
        try {
            c.fn();
            std::printf("ok\n");
        } catch (const Failure &f) {
            failed++;
            std::printf("FAIL\n    %s\n", f.msg.c_str());
        } catch (const std::exception &e) {
            failed++;
            std::printf("FAIL\n    exception: %s\n", e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%d run, %d failed (%s)\n", run, failed, g_device ? "device" : "host");
    g_backend.reset();
    return failed == 0 && run > 0 ? 0 : 1;
}
