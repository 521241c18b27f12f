/*
 * glint_attn.h -- C ABI of the MI355X (gfx950) attention path for Glint.
 *
 * This library replaces the attention step of Glint's GPU backend and its
 * CPU flash-attention fallback:
 *   - GpuBackend::attention / attention_resident   src/backend/gpu.rs:266-397, :860-992
 *   - GpuBackend::create_kv_cache / GpuKvCache      src/backend/gpu.rs:1039-1104
 *   - KvStore::write / export_raw / import_raw      src/cache/mod.rs:24-109
 *   - PagePool page recycle and copy-on-write       src/cache/paged.rs:79-82, :433-444
 *   - attn_heads_cpu over a batch (decode)          src/transformer/forward.rs:1468-1502
 *   - prefill attention loop                        src/transformer/forward.rs:927-958
 * and, beside it on a decode step, RoPE (src/tensor/ops.rs:212-245) and the
 * Q8_0 weight matvec (src/tensor/quantized.rs:247-346, :587-610).
 * The numerics follow flash_attn_1d_ext (src/tensor/flash.rs:46-124).
 *
 * Conventions (the same as Glint's outbound C API, include/glint.h:21-35):
 *   - Every function returns an int status: GLA_OK (0) or a negative code.
 *     gla_last_error() returns a thread-local message for the last failure on
 *     the calling thread. No C++ exception crosses the boundary.
 *   - Handles are not thread-safe; use one gla_ctx per thread or lock.
 *   - "Device" pointers are HIP device addresses on the context's device;
 *     "host" pointers are ordinary memory borrowed for the call only.
 *   - Device-pointer entry points are asynchronous on the context's stream;
 *     gla_sync() waits for them. Host-pointer entry points return after the
 *     results are in host memory.
 *   - Unsupported shapes return GLA_ERR_INVALID so the caller can take its
 *     CPU path, as it does for the wgpu MAX_SEQ guard (src/backend/gpu.rs:277-282).
 *
 * Supported shapes: head_dim in {64, 128, 256}; any n_heads that is a
 * multiple of n_kv_heads; any context length (no MAX_SEQ limit).
 */
#ifndef GLINT_ATTN_H
#define GLINT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The GPU ones correspond to GlintError (src/error.rs:41-52, :78-82). */
#define GLA_OK 0
#define GLA_ERR_NO_DEVICE (-1)      /* GlintError::GpuAdapterNotFound */
#define GLA_ERR_DEVICE (-2)         /* GlintError::GpuDeviceError */
#define GLA_ERR_BUFFER (-3)         /* GlintError::GpuBufferError (alloc / copy) */
#define GLA_ERR_KERNEL (-4)         /* GlintError::GpuShaderError (launch) */
#define GLA_ERR_INVALID (-5)        /* bad argument or unsupported shape */
#define GLA_ERR_POOL_EXHAUSTED (-6) /* GlintError::KvPagePoolExhausted */

/* Positions per page -- src/cache/paged.rs:55 PAGE_SIZE. */
#define GLA_PAGE_SIZE 16

/* KV element formats: KvCache / PagedKvCache (f32) and KvCacheQ8 (Q8_0,
 * 32-element blocks with one f16 scale, src/cache/mod.rs:263-315). */
typedef enum gla_kv_dtype { GLA_KV_F32 = 0, GLA_KV_Q8_0 = 1 } gla_kv_dtype;

/* Arithmetic of the prefill matrix products. */
typedef enum gla_precision {
    GLA_PREC_F32 = 0, /* fp32 inputs, fp32-accumulate MFMA */
    GLA_PREC_BF16 = 1 /* bf16-rounded Q/K/P/V inputs, fp32-accumulate MFMA */
} gla_precision;

typedef struct gla_ctx gla_ctx;
typedef struct gla_kv gla_kv;

/* ---- context ------------------------------------------------------------ */

/* Thread-local message of the last failed call on this thread ("" if none).
 * Replaces glint_last_error (include/glint.h, src/ffi/mod.rs:64). */
const char *gla_last_error(void);

/* Open `device`. Returns GLA_ERR_NO_DEVICE when no HIP device is present,
 * the condition GpuBackend::new reports as GpuAdapterNotFound
 * (src/backend/gpu.rs:44-56); the caller then stays on its CPU path. */
int gla_create(int device, gla_ctx **out);
/* Frees the context and the device memory of every cache, pool and weight
 * set created on it; their handles must still be released
 * (gla_kv_destroy, gla_q8w_destroy), which then frees only the handle, and
 * any other use of them fails with GLA_ERR_INVALID. */
int gla_destroy(gla_ctx *ctx);

/* Run subsequent work on `hip_stream` (a hipStream_t); NULL restores the
 * context's own stream. Each stream the context has launched work on has
 * its own device scratch (decode split partials, bf16 prefill tile images,
 * matvec activation pieces), so calls queued on different streams at once
 * never share it and may overlap; calls on one stream run in order as usual.
 * That scratch is held until gla_destroy or gla_release_stream. The stream
 * must outlive its use by the context: switch away from it (or release it)
 * before destroying it. The context itself is not thread-safe: switch
 * streams from one thread. */
int gla_set_stream(gla_ctx *ctx, void *hip_stream);
/* The hipStream_t work is enqueued on. */
void *gla_get_stream(gla_ctx *ctx);
/* Free the device scratch the context keeps for `hip_stream` (split
 * partials, tile images, matvec pieces), after waiting for that stream.
 * Scratch is otherwise held per stream until gla_destroy, so a caller that
 * makes a stream per request calls this before destroying each stream. If
 * `hip_stream` is the current stream, the context first returns to its own
 * stream. Graphs captured on `hip_stream` must not be replayed afterwards.
 * Buffers that a stream's scratch outgrew stay allocated until gla_destroy
 * (earlier graphs may address them). Releasing a stream the context never
 * used is a no-op. */
int gla_release_stream(gla_ctx *ctx, void *hip_stream);
/* Wait for all work enqueued on the context's stream. */
int gla_sync(gla_ctx *ctx);
/* Number of compute units of the context's device (0 on error). */
int gla_device_cu_count(gla_ctx *ctx);


/* ---- device memory (for device-resident q / out / tables) --------------- */

int gla_dev_alloc(gla_ctx *ctx, size_t bytes, void **out);
int gla_dev_free(gla_ctx *ctx, void *ptr);
/* Host -> device; returns once `src` may be reused. */
int gla_memcpy_htod(gla_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);
/* Device -> host; waits for the context's stream first. */
int gla_memcpy_dtoh(gla_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes);

/* ---- KV storage ---------------------------------------------------------- */

/* Contiguous caches for n_seqs sequences: each holds max_seq_len positions of
 * every layer, like KvCache::new / KvCacheQ8::new (src/cache/mod.rs:127-140,
 * :288-294) and GpuBackend::create_kv_cache (src/backend/gpu.rs:1060-1104).
 * Storage is zero-initialised. */
int gla_kv_cache_create(gla_ctx *ctx, gla_kv_dtype dtype, int n_seqs, int n_layers, int max_seq_len,
                        int n_kv_heads, int head_dim, gla_kv **out);

/* A pool of capacity_pages pages; a page holds GLA_PAGE_SIZE positions of K
 * and V of one layer and has no layer identity, like PagePool::preallocated
 * (src/cache/paged.rs:176-189). Page ids run 0 .. capacity_pages-1; the caller
 * keeps the page tables and reference counts (PagedKvCache's table[layer][page],
 * src/cache/paged.rs:254-260). Storage is zero-initialised. */
int gla_pool_create(gla_ctx *ctx, gla_kv_dtype dtype, int n_kv_heads, int head_dim, int capacity_pages,
                    gla_kv **out);

int gla_kv_destroy(gla_kv *kv);

/* Row id of (seq, layer, pos) in a contiguous cache; row ids of a pool are
 * page * GLA_PAGE_SIZE + slot. Returns -1 on a bad argument. */
int64_t gla_kv_row_id(const gla_kv *kv, int seq, int layer, int pos);

/* Write K and V rows (kv_dim = n_kv_heads * head_dim floats each) -- the
 * KvStore::write analogue (src/cache/mod.rs:166-177, :374-388,
 * src/cache/paged.rs:467-490). Q8_0 storage quantises on write with the
 * rules of KvCacheQ8::quantize_into (src/cache/mod.rs:296-315), bit-exactly.
 * Device pointers; asynchronous. rows: int64[n_rows]; k, v: [n_rows][kv_dim].
 * The rows are written in parallel: ids repeated within one call leave one
 * of their rows (which one is unspecified), and ids outside the storage are
 * skipped on the device. */
int gla_kv_write_rows(gla_ctx *ctx, gla_kv *kv, const int64_t *rows_dev, const float *k_dev,
                      const float *v_dev, int n_rows);
/* The same with host pointers; returns when the rows are written. */
int gla_kv_write_rows_host(gla_ctx *ctx, gla_kv *kv, const int64_t *rows, const float *k, const float *v,
                           int n_rows);

/* Export rows as the bytes KvStore::export_raw produces for them
 * (src/cache/mod.rs:68-84, :219-241, :390-395): f32 rows are kv_dim native
 * floats; Q8_0 rows are ceil(kv_dim/32) blocks of [f16 scale LE][32 x i8].
 * Host pointers; k_out and v_out receive n_rows * row_bytes each. */
int gla_kv_export_rows_host(gla_ctx *ctx, const gla_kv *kv, const int64_t *rows, int n_rows, uint8_t *k_out,
                            uint8_t *v_out);
/* Inverse of export (KvStore::import_raw, src/cache/mod.rs:397-422):
 * stores the bytes as they are (Q8_0 blocks are not re-quantised). */
int gla_kv_import_rows_host(gla_ctx *ctx, gla_kv *kv, const int64_t *rows, int n_rows, const uint8_t *k_in,
                            const uint8_t *v_in);
/* Bytes one exported K (or V) row occupies. */
int64_t gla_kv_row_bytes(const gla_kv *kv);

/* Copy-on-write of a shared page (src/cache/paged.rs:433-444) and the
 * recycled-page wipe (PageBuf::reset, src/cache/paged.rs:79-82). Pools only;
 * asynchronous. */
int gla_pool_copy_page(gla_ctx *ctx, gla_kv *pool, int src_page, int dst_page);
int gla_pool_zero_page(gla_ctx *ctx, gla_kv *pool, int page);

/* ---- attention ----------------------------------------------------------- */

/* window_start of src/transformer/forward.rs:574-581: 0 on odd layers when
 * `alternating` (Gemma-2), else max(0, pos - sliding_window + 1) when
 * sliding_window > 0, else 0. attend_len is then pos + 1 - window_start. */
long gla_window_start(long pos, long sliding_window, int alternating, int layer);

/* Batched single-token decode: for every sequence b and q-head h,
 *   out[b][h] = softmax_j(cap(q[b][h] . K[j] * scale)) . V[j]
 * over positions j in [kv_start[b], kv_start[b] + kv_len[b]) of the sequence's
 * KV, K/V head h / (n_heads / n_kv_heads), cap(s) = softcap * tanh(s / softcap)
 * when softcap > 0 -- flash_attn_1d_ext per head (src/tensor/flash.rs:46-124)
 * as attn_heads_cpu calls it (src/transformer/forward.rs:240-270). kv_len 0
 * gives a zero output, as the reference's pre-zeroed buffer does. Non-finite
 * data behaves as there: a NaN reaching a head's weights or sums makes the
 * head's output NaN (the reference leaves such sums unnormalised,
 * flash.rs:118-123), and an infinite value under a non-zero weight gives
 * +-inf in its dimension.
 *
 * Out-of-range indices. The reference panics on a position or page id
 * outside the storage (Vec indexing in PagedKvCache::read_k_head,
 * src/cache/paged.rs:453-465; the write/truncate bounds of
 * src/cache/mod.rs:167-171, :186-190). Here:
 *   - with the host copies (kv_start_host / kv_len_host), every window is
 *     checked on the host before anything is launched: kv_start < 0,
 *     kv_len < 0, kv_len > max_kv_len, or kv_start + kv_len past the
 *     storage (the cache's max_seq; a pool's page_table_stride * 16
 *     positions) returns GLA_ERR_INVALID and the next call works;
 *   - the device arrays themselves are not read by the host. The kernels
 *     clamp every index they derive from them into the storage (positions
 *     to [0, storage positions), seq_slot to [0, n_seqs of the cache), page
 *     ids to [0, pages of the pool)), so a malformed device length, slot or
 *     page-table entry gives attention over the clamped positions and
 *     GLA_OK, never an access outside the storage. */
typedef struct gla_decode_args {
    const gla_kv *kv;          /* contiguous cache or pool */
    int layer;                 /* contiguous caches: layer to read; ignored for pools */
    int n_seqs;                /* batch size B */
    const int32_t *seq_slot;   /* caches: device int32[B], cache sequence read by batch row b
                                  (NULL: row b reads sequence b) */
    const int32_t *page_table; /* pools: device int32[B][page_table_stride], the physical page
                                  of each logical page pos / GLA_PAGE_SIZE (this layer's table) */
    int page_table_stride;
    const int32_t *kv_start; /* device int32[B]: window_start */
    const int32_t *kv_len;   /* device int32[B]: attend_len (>= 0) */
    int max_kv_len;          /* host: >= every kv_len[b] (sizes the launch) */
    int n_heads;
    float scale;   /* query_pre_attn_scalar or 1/sqrt(head_dim) (forward.rs:583-585) */
    float softcap; /* attn_logit_softcapping; <= 0 means none */
    const float *q; /* device [B][n_heads][head_dim] */
    float *out;     /* device [B][n_heads][head_dim] */
    /* Optional host copies of kv_start / kv_len: both NULL, or both int32[B]
     * holding the values of the device arrays. Read during the call only, to
     * size the launch to the batch's real lengths (the engine keeps every
     * sequence's position on the host, src/transformer/forward.rs:1468-1507,
     * so passing them is free); without them the launch is sized for
     * max_kv_len. */
    const int32_t *kv_start_host;
    const int32_t *kv_len_host;
} gla_decode_args;

int gla_decode(gla_ctx *ctx, const gla_decode_args *args);

/* Device scratch gla_decode_noalloc may use, in bytes (one array per GPU). */
#define GLA_DECODE_NOALLOC_SCRATCH_BYTES (16u << 20)
/* (sequence, KV head, head group) units an f32-storage gla_decode_noalloc
 * call may hold (arrival counters of the short-window merge; one array per
 * GPU). Never the tighter limit: a unit that counts arrivals has at least
 * two split partials of at least 384 bytes each, so the partial scratch
 * refuses a call before it reaches 21,846 such units. */
#define GLA_DECODE_NOALLOC_UNITS 65536

/* gla_decode that allocates nothing. It has no counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and bit-identical results as gla_decode; the split
 * partials live in a static device array of GLA_DECODE_NOALLOC_SCRATCH_BYTES
 * that each GPU the library runs on holds until the process ends (resolved
 * once per device by gla_create). A call whose partials need more returns
 * GLA_ERR_INVALID before anything is launched. The capacity depends on the
 * storage: at Llama-3-8B heads (32/8, d128) and 8,192 positions per
 * sequence, Q8_0 storage takes up to 192 sequences per call (B=64 needs
 * 5.3 MiB), f32 storage up to 29 (f32 splits are shorter: 33 partials per
 * KV head against 5). Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (two streams or two contexts) race. Nothing in it
 * needs clearing: a call writes every partial it reads. f32 windows of at
 * most 65 pages (33 at head groups of over 512 floats) merge their splits in
 * the last workgroup to finish and count arrivals in a second static array of GLA_DECODE_NOALLOC_UNITS counters
 * (zero when the library loads, left at zero by every call); a call with
 * more (sequence, KV head, head group) units returns GLA_ERR_INVALID. */
int gla_decode_noalloc(gla_ctx *ctx, const gla_decode_args *args);

/* Batched causal prefill: query row r of sequence b sits at absolute
 * position pos_offset[b] + (r - q_start[b]) and attends positions
 * [w, that position] of the sequence's KV, w = max(0, pos - sliding_window + 1)
 * when sliding_window > 0 else 0 -- the loop of src/transformer/forward.rs:927-958
 * (pass sliding_window = 0 for a global layer of an alternating model). The
 * K/V of every attended position must already be written, as the reference
 * writes the chunk before attending (forward.rs:874-877).
 *
 * Out-of-range indices, as for gla_decode: the attended key positions are
 * clamped into the storage (a pos_offset past it attends the stored
 * positions only; a negative one attends none of its own) and seq_slot and
 * page-table entries into the cache or pool, so a malformed device value
 * gives clamped attention and GLA_OK where the reference would panic. The
 * query rows q_start[b] .. q_start[b+1]-1 index q and out, whose size the
 * library is not told: they must lie inside those buffers. */
typedef struct gla_prefill_args {
    const gla_kv *kv;
    int layer;
    int n_seqs;
    const int32_t *seq_slot;   /* caches: device int32[B] or NULL */
    const int32_t *page_table; /* pools: device int32[B][page_table_stride] */
    int page_table_stride;
    const int32_t *q_start;    /* device int32[B + 1]: query rows of b are q_start[b] .. q_start[b+1]-1 */
    const int32_t *pos_offset; /* device int32[B] */
    int max_q_len;             /* host: >= every q_start[b+1] - q_start[b] */
    int n_heads;
    float scale;
    float softcap;          /* <= 0: none */
    int sliding_window;     /* <= 0: none */
    gla_precision precision;
    const float *q; /* device [total_rows][n_heads][head_dim] */
    float *out;     /* device [total_rows][n_heads][head_dim] */
} gla_prefill_args;

int gla_prefill(gla_ctx *ctx, const gla_prefill_args *args);

/* Host-buffer mirror of GpuBackend::attention (src/backend/gpu.rs:266-397):
 * q [n_heads][head_dim]; k, v [seq_len][n_kv_heads][head_dim]; out
 * [n_heads][head_dim]. Adds the soft-cap the wgpu shader lacks and has no
 * MAX_SEQ limit. Returns when `out` is filled. */
int gla_attention(gla_ctx *ctx, const float *q, const float *k, const float *v, int n_heads, int n_kv_heads,
                  int head_dim, int seq_len, float scale, float softcap, float *out);

/* Host-buffer mirror of GpuBackend::attention_resident
 * (src/backend/gpu.rs:860-992) over a device-resident contiguous cache:
 * attends [window_start, window_start + attend_len) of (seq, layer). */
int gla_attention_resident(gla_ctx *ctx, const float *q, const gla_kv *cache, int seq, int layer,
                           int window_start, int attend_len, int n_heads, float scale, float softcap,
                           float *out);

/* ---- the ops beside attention on a decode step --------------------------- */

/* RoPE in place, ops::rope (src/tensor/ops.rs:212-245) on device rows:
 * x [n_rows][n_heads][head_dim], row r at position pos[r] (device int32).
 * For even i < min(rot_dim, head_dim) & ~1 every head's pair (i, i+1) is
 * rotated by (pos / scaling_factor) * (1 / powf(freq_base, i / head_dim)),
 * the frequency taken from the host's powf as the reference's f32::powf
 * takes it; the other dimensions are left as they are. Like the reference,
 * freq_base and scaling_factor are not validated. Asynchronous; no device
 * allocation or copy (the frequencies travel as kernel arguments). */
int gla_rope(gla_ctx *ctx, float *x, int n_rows, int n_heads, int head_dim, const int32_t *pos, float freq_base,
             float scaling_factor, int rot_dim);

/* Q8_0 weights on the device, uploaded once: the GpuBackend::upload_buffer of
 * a GGML Q8_0 tensor (src/backend/gpu.rs:111-121), repacked for the MFMA
 * matvec. ggml_host: rows x (cols / 32) blocks of [f16 scale LE][32 x i8]
 * (34 bytes); cols a multiple of 32. Returns when the weights are on the
 * device. */
typedef struct gla_q8w gla_q8w;
int gla_q8w_create(gla_ctx *ctx, const uint8_t *ggml_host, int rows, int cols, gla_q8w **out);
int gla_q8w_destroy(gla_q8w *w);
int gla_q8w_rows(const gla_q8w *w);
int gla_q8w_cols(const gla_q8w *w);

/* y[v][r] = sum_c W[r][c] * x[v][c] for n_vec vectors: QuantizedTensor::matvec
 * and matvec_batch over Q8_0 (src/tensor/quantized.rs:247-346, :587-610; the
 * wgpu matvec_q8_0 shader's job). x device [n_vec][cols], y device
 * [n_vec][rows], f32. Asynchronous; the weights are read once per 64
 * vectors. n_vec above 262,128 is refused (GLA_ERR_INVALID): split the call. */
int gla_matvec_q8_0(gla_ctx *ctx, const gla_q8w *w, const float *x, int n_vec, float *y);

#ifdef __cplusplus
}
#endif

#endif /* GLINT_ATTN_H */
