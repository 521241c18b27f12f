// gla_kvstore.hip -- device side of KvStore::write / export_raw / import_raw
// and of the page pool's copy-on-write and recycle wipe.
//
// Quantize-on-write reproduces KvCacheQ8::quantize_into (src/cache/mod.rs:296-315)
// bit for bit: d = max|x| / 127 (1.0 for an all-zero block), q = clamp(round
// half away from zero(x * (1/d)), -127, 127) computed from the f32 d, NaN -> 0,
// and the stored scale is f16(d) rounded to nearest even.
#include "gla_internal.h"

namespace gla {

namespace {

struct RowOps {
    KvLayout L;
    int64_t n_rows_total;  // valid row ids are [0, n_rows_total)
    int head_dim;
    int kv_dim;
    int n_blocks;  // kv_dim / 32
    bool q8;
};

RowOps row_ops(const gla_kv *kv) {
    RowOps o;
    o.L = layout_of(kv);
    o.n_rows_total = kv->n_pages * GLA_PAGE_SIZE;
    o.head_dim = kv->head_dim;
    o.kv_dim = kv->kv_dim;
    o.n_blocks = kv->kv_dim / 32;
    o.q8 = kv->dtype == GLA_KV_Q8_0;
    return o;
}

// Byte offset of element `gi` (0 .. kv_dim-1) of row `row`, and of its scale.
__device__ __forceinline__ int64_t elem_off(const RowOps &o, int64_t row, int gi, int esize) {
    const int64_t page = row >> 4;
    const int slot = (int)(row & 15);
    const int h = gi / o.head_dim;
    const int e = gi - h * o.head_dim;
    return page * o.L.page_stride + (int64_t)h * o.L.head_stride + (int64_t)slot * o.L.row_stride +
           (int64_t)e * esize;
}
// Byte offset of the Q8_0 scale of (row, element gi) from L.ks (which = 0,
// parity-grouped) or L.vs (which = 1, row-major).
__device__ __forceinline__ int64_t scale_off(const RowOps &o, int64_t row, int gi, int which) {
    const int64_t page = row >> 4;
    const int slot = (int)(row & 15);
    const int h = gi / o.head_dim;
    const int e = gi - h * o.head_dim;
    const int idx = which ? slot * (o.head_dim >> 5) + (e >> 5) : q8ks_off(slot, e >> 5, o.head_dim);
    return page * o.L.page_stride + (int64_t)h * o.L.head_stride + (int64_t)idx * 2;
}

// Byte offset of Q8_0 quant (row, element gi) of K (which = 0) or V (1); the
// quants of a (page, head) are stored in MFMA operand order (q8k_off / q8v_off).
__device__ __forceinline__ int64_t q8_off(const RowOps &o, int64_t row, int gi, int which) {
    const int64_t page = row >> 4;
    const int slot = (int)(row & 15);
    const int h = gi / o.head_dim;
    const int e = gi - h * o.head_dim;
    const int in_head = which ? q8v_off(slot, e, o.head_dim) : q8k_off(slot, e, o.head_dim);
    return page * o.L.page_stride + (int64_t)h * o.L.head_stride + in_head;
}

__device__ __forceinline__ int8_t quantize_one(float x, float inv_d) {
    float r = roundf(x * inv_d);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (r != r) ? (int8_t)0 : (int8_t)r;
}

// grid.x = rows, threads loop over (K|V, block of 32 elements)
__global__ __launch_bounds__(64) void write_rows_kernel(const RowOps o, const int64_t *rows, const float *k,
                                                        const float *v, int n) {
    const int r = blockIdx.x;
    if (r >= n) return;
    const int64_t row = rows[r];
    if (row < 0 || row >= o.n_rows_total) return;
    uint8_t *kbase = const_cast<uint8_t *>(o.L.k);
    uint8_t *vbase = const_cast<uint8_t *>(o.L.v);
    for (int t = threadIdx.x; t < 2 * o.n_blocks; t += blockDim.x) {
        const int which = t >= o.n_blocks;
        const int blk = which ? t - o.n_blocks : t;
        const float *src = (which ? v : k) + (int64_t)r * o.kv_dim + blk * 32;
        uint8_t *dst = which ? vbase : kbase;
        const int gi0 = blk * 32;
        if (!o.q8) {
            float *d = reinterpret_cast<float *>(dst + elem_off(o, row, gi0, 4));
#pragma unroll
            for (int j = 0; j < 32; j += 4) *reinterpret_cast<float4 *>(d + j) = *reinterpret_cast<const float4 *>(src + j);
        } else {
            float x[32];
#pragma unroll
            for (int j = 0; j < 32; j += 4) {
                float4 f = *reinterpret_cast<const float4 *>(src + j);
                x[j] = f.x;
                x[j + 1] = f.y;
                x[j + 2] = f.z;
                x[j + 3] = f.w;
            }
            float max_abs = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; j++) max_abs = fmaxf(max_abs, fabsf(x[j]));
            const float dsc = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
            const float inv_d = 1.0f / dsc;
            uint32_t w[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint32_t b0 = (uint8_t)quantize_one(x[4 * j + 0], inv_d);
                uint32_t b1 = (uint8_t)quantize_one(x[4 * j + 1], inv_d);
                uint32_t b2 = (uint8_t)quantize_one(x[4 * j + 2], inv_d);
                uint32_t b3 = (uint8_t)quantize_one(x[4 * j + 3], inv_d);
                w[j] = (b0 | (b1 << 8) | (b2 << 16) | (b3 << 24)) ^ 0x80808080u;  // stored as x + 128
            }
            if (!which) {  // K: four 8-byte runs (d = gi0 + 8*kg .. +7)
#pragma unroll
                for (int kg = 0; kg < 4; kg++)
                    *reinterpret_cast<uint2 *>(dst + q8_off(o, row, gi0 + 8 * kg, 0)) = make_uint2(w[2 * kg], w[2 * kg + 1]);
            } else {  // V: one byte per element, 4-position columns
#pragma unroll
                for (int j = 0; j < 32; j++) dst[q8_off(o, row, gi0 + j, 1)] = (uint8_t)(w[j >> 2] >> ((j & 3) * 8));
            }
            uint8_t *sb = const_cast<uint8_t *>(which ? o.L.vs : o.L.ks);
            *reinterpret_cast<uint16_t *>(sb + scale_off(o, row, gi0, which)) = __half_as_ushort(__float2half_rn(dsc));
        }
    }
}

// Export to Glint's row bytes (f32 rows, or Q8_0 34-byte blocks).
__global__ __launch_bounds__(64) void export_rows_kernel(const RowOps o, const int64_t *rows, int n,
                                                         uint8_t *k_out, uint8_t *v_out) {
    const int r = blockIdx.x;
    if (r >= n) return;
    const int64_t row = rows[r];
    if (row < 0 || row >= o.n_rows_total) return;
    const int64_t row_bytes = o.q8 ? (int64_t)o.n_blocks * 34 : (int64_t)o.kv_dim * 4;
    for (int t = threadIdx.x; t < 2 * o.n_blocks; t += blockDim.x) {
        const int which = t >= o.n_blocks;
        const int blk = which ? t - o.n_blocks : t;
        const uint8_t *src = which ? o.L.v : o.L.k;
        uint8_t *out = (which ? v_out : k_out) + (int64_t)r * row_bytes;
        const int gi0 = blk * 32;
        if (!o.q8) {
            const uint8_t *s = src + elem_off(o, row, gi0, 4);
            for (int j = 0; j < 128; j++) out[(int64_t)gi0 * 4 + j] = s[j];
        } else {
            const uint8_t *sc = (which ? o.L.vs : o.L.ks) + scale_off(o, row, gi0, which);
            uint8_t *ob = out + (int64_t)blk * 34;
            ob[0] = sc[0];
            ob[1] = sc[1];
            for (int j = 0; j < 32; j++) ob[2 + j] = src[q8_off(o, row, gi0 + j, which)] ^ 0x80;
        }
    }
}

__global__ __launch_bounds__(64) void import_rows_kernel(const RowOps o, const int64_t *rows, int n,
                                                         const uint8_t *k_in, const uint8_t *v_in) {
    const int r = blockIdx.x;
    if (r >= n) return;
    const int64_t row = rows[r];
    if (row < 0 || row >= o.n_rows_total) return;
    const int64_t row_bytes = o.q8 ? (int64_t)o.n_blocks * 34 : (int64_t)o.kv_dim * 4;
    for (int t = threadIdx.x; t < 2 * o.n_blocks; t += blockDim.x) {
        const int which = t >= o.n_blocks;
        const int blk = which ? t - o.n_blocks : t;
        uint8_t *dst = const_cast<uint8_t *>(which ? o.L.v : o.L.k);
        const uint8_t *in = (which ? v_in : k_in) + (int64_t)r * row_bytes;
        const int gi0 = blk * 32;
        if (!o.q8) {
            uint8_t *d = dst + elem_off(o, row, gi0, 4);
            for (int j = 0; j < 128; j++) d[j] = in[(int64_t)gi0 * 4 + j];
        } else {
            uint8_t *sc = const_cast<uint8_t *>(which ? o.L.vs : o.L.ks) + scale_off(o, row, gi0, which);
            const uint8_t *ib = in + (int64_t)blk * 34;
            sc[0] = ib[0];
            sc[1] = ib[1];
            for (int j = 0; j < 32; j++) dst[q8_off(o, row, gi0 + j, which)] = ib[2 + j] ^ 0x80;
        }
    }
}

// Page-granular copy and fill with 16-byte vectors (no hipMemsetAsync, so the
// calls stay valid inside a captured graph).
__global__ __launch_bounds__(256) void copy_bytes_kernel(const uint4 *src, uint4 *dst, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// Fill of whole pages: a 16-byte unit at byte offset o of its (page, head)
// block of `head16` units gets `quant` below unit `quant16`, zero above (f32
// pages: everything zero; Q8_0 pages: quants 0x80 = stored 0, scales 0).
__global__ __launch_bounds__(256) void zero_bytes_kernel(uint4 *dst, int64_t n16, int64_t head16, int64_t quant16,
                                                         uint32_t quant) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t w = (i % head16) < quant16 ? quant : 0u;
        dst[i] = make_uint4(w, w, w, w);
    }
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "%s launch: %s", what, hipGetErrorString(e));
    return GLA_OK;
}

unsigned grid_for(int64_t n16) {
    int64_t blocks = (n16 + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    return (unsigned)blocks;
}

}  // namespace

int launch_write_rows(gla_ctx *ctx, gla_kv *kv, const int64_t *rows, const float *k, const float *v, int n) {
    if (n <= 0) return GLA_OK;
    const RowOps o = row_ops(kv);
    hipLaunchKernelGGL(write_rows_kernel, dim3(n), dim3(64), 0, ctx->stream, o, rows, k, v, n);
    return check_launch("write_rows_kernel");
}

int launch_export_rows(gla_ctx *ctx, const gla_kv *kv, const int64_t *rows, int n, uint8_t *k_out,
                       uint8_t *v_out) {
    if (n <= 0) return GLA_OK;
    const RowOps o = row_ops(kv);
    hipLaunchKernelGGL(export_rows_kernel, dim3(n), dim3(64), 0, ctx->stream, o, rows, n, k_out, v_out);
    return check_launch("export_rows_kernel");
}

int launch_import_rows(gla_ctx *ctx, gla_kv *kv, const int64_t *rows, int n, const uint8_t *k_in,
                       const uint8_t *v_in) {
    if (n <= 0) return GLA_OK;
    const RowOps o = row_ops(kv);
    hipLaunchKernelGGL(import_rows_kernel, dim3(n), dim3(64), 0, ctx->stream, o, rows, n, k_in, v_in);
    return check_launch("import_rows_kernel");
}

int launch_copy_page(gla_ctx *ctx, gla_kv *kv, int64_t src, int64_t dst) {
    const int64_t n16 = kv->page_bytes / 16;
    const uint4 *s = reinterpret_cast<const uint4 *>(kv->base + src * kv->page_bytes);
    uint4 *d = reinterpret_cast<uint4 *>(kv->base + dst * kv->page_bytes);
    hipLaunchKernelGGL(copy_bytes_kernel, dim3(grid_for(n16)), dim3(256), 0, ctx->stream, s, d, n16);
    return check_launch("copy_bytes_kernel");
}

int launch_zero_pages(gla_ctx *ctx, gla_kv *kv, int64_t first, int64_t count) {
    const int64_t n16 = kv->page_bytes / 16 * count;
    const int64_t head16 = kv->head_bytes / 16;
    const bool q8 = kv->dtype == GLA_KV_Q8_0;
    const int64_t quant16 = q8 ? (int64_t)GLA_PAGE_SIZE * kv->head_dim * 2 / 16 : 0;  // Kq and Vq
    uint4 *d = reinterpret_cast<uint4 *>(kv->base + first * kv->page_bytes);
    hipLaunchKernelGGL(zero_bytes_kernel, dim3(grid_for(n16)), dim3(256), 0, ctx->stream, d, n16, head16, quant16,
                       0x80808080u);
    return check_launch("zero_bytes_kernel");
}

}  // namespace gla
