// host_page_store.hpp -- a PageStore in host memory (f32 pages), test
// infrastructure only: it lets the page bookkeeping of PagePool /
// PagedKvCache (refcounts, copy-on-write, recycling, exhaustion) run in the
// CPU test suite. It stores and copies bytes; it computes no attention.
#pragma once

#include <cstring>
#include <vector>

#include "glint.hpp"

namespace glint_test {

class HostPageStore final : public glint::PageStore {
  public:
    HostPageStore(size_t capacity, size_t n_kv_heads, size_t head_dim)
        : cap_(capacity), nkv_(n_kv_heads), hd_(head_dim),
          k_(capacity * glint::PAGE_SIZE * n_kv_heads * head_dim, 0.0f),
          v_(capacity * glint::PAGE_SIZE * n_kv_heads * head_dim, 0.0f) {}
    size_t capacity() const override { return cap_; }
    size_t n_kv_heads() const override { return nkv_; }
    size_t head_dim() const override { return hd_; }
    gla_kv_dtype dtype() const override { return GLA_KV_F32; }
    size_t row_bytes() const override { return kv_dim() * sizeof(float); }
    glint::Status write_rows(const int64_t *rows, size_t n, const float *k, const float *v) override {
        for (size_t i = 0; i < n; i++) {
            if (!in_range(rows[i])) return glint::GlintError::gpu_buffer_error("row out of range");
            std::memcpy(&k_[rows[i] * kv_dim()], k + i * kv_dim(), row_bytes());
            std::memcpy(&v_[rows[i] * kv_dim()], v + i * kv_dim(), row_bytes());
        }
        return {};
    }
    glint::Status export_rows(const int64_t *rows, size_t n, uint8_t *k, uint8_t *v) const override {
        for (size_t i = 0; i < n; i++) {
            if (!in_range(rows[i])) return glint::GlintError::gpu_buffer_error("row out of range");
            std::memcpy(k + i * row_bytes(), &k_[rows[i] * kv_dim()], row_bytes());
            std::memcpy(v + i * row_bytes(), &v_[rows[i] * kv_dim()], row_bytes());
        }
        return {};
    }
    glint::Status import_rows(const int64_t *rows, size_t n, const uint8_t *k, const uint8_t *v) override {
        for (size_t i = 0; i < n; i++) {
            if (!in_range(rows[i])) return glint::GlintError::gpu_buffer_error("row out of range");
            std::memcpy(&k_[rows[i] * kv_dim()], k + i * row_bytes(), row_bytes());
            std::memcpy(&v_[rows[i] * kv_dim()], v + i * row_bytes(), row_bytes());
        }
        return {};
    }
    glint::Status copy_page(size_t src, size_t dst) override {
        const size_t n = glint::PAGE_SIZE * kv_dim();
        std::memcpy(&k_[dst * n], &k_[src * n], n * sizeof(float));
        std::memcpy(&v_[dst * n], &v_[src * n], n * sizeof(float));
        copies++;
        return {};
    }
    glint::Status zero_page(size_t page) override {
        const size_t n = glint::PAGE_SIZE * kv_dim();
        std::fill(k_.begin() + page * n, k_.begin() + (page + 1) * n, 0.0f);
        std::fill(v_.begin() + page * n, v_.begin() + (page + 1) * n, 0.0f);
        wipes++;
        return {};
    }
    size_t copies = 0, wipes = 0;

  private:
    bool in_range(int64_t r) const { return r >= 0 && (size_t)r < cap_ * glint::PAGE_SIZE; }
    size_t cap_, nkv_, hd_;
    std::vector<float> k_, v_;
};

}  // namespace glint_test
