// gla_internal.h -- shared definitions of the gfx950 attention library.
//
// Device layout of KV storage (contiguous caches and pools alike).
// Everything is a page of GLA_PAGE_SIZE (16) positions of one layer; a
// contiguous cache of (n_seqs, n_layers, max_seq) is the page range
//   page = (seq * n_layers + layer) * pages_per_layer + pos / 16
// so one kernel family reads both. Within a page the heads are contiguous
// chunks ("head-major"), so one (page, kv head) is a single span of HBM:
//
//   f32 : [page][kv_head] { K[16][d] f32 | V[16][d] f32 }            128*d B per head
//   Q8_0: [page][kv_head] { Kq[16][d] i8 | Vq[16][d] i8 |
//                           Ks[16][d/32] f16 | Vs[16][d/32] f16 }    34*d B per head
//
// The Q8_0 split of quants and scales keeps every quant access 16-byte
// aligned (Glint's 34-byte block, src/cache/mod.rs:276, is not); the byte
// count per position is unchanged (34 per 32 elements) and export re-packs
// the blocks.
//
// Q8_0 quants are stored as x + 128 (sign bit flipped; a zeroed page holds
// 0x80 bytes) in the order the MFMA decode kernel consumes them (q8k_off /
// q8v_off below). A (page, head) K or V block is D/64 pieces of 1 KB; lane l
// of a wave finds its 16 operand bytes of piece c at c*1024 + l*16, so one
// 16-byte-per-lane load moves a contiguous kilobyte.
//   K[slot t][d]: lane (kg = (d>>3)&3)*16 + t holds, for each 32-block
//                 blk = d>>5, the 8 bytes d = blk*32 + kg*8 + 0..7
//                 (piece blk>>1, bytes (blk&1)*8 ..).
//   V[slot s][d]: lane (s>>2)*16 + (d&15) holds, for each 16-wide d tile
//                 dt = d>>4, the 4 bytes of slots (s & ~3) + 0..3
//                 (piece dt>>2, bytes (dt&3)*4 ..).
// K scales are grouped by block parity, Ks[blk & 1][slot][blk >> 1]
// (q8ks_off), V scales are row-major, Vs[slot][blk], all f16.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <utility>
#include <vector>

#include "../../include/glint_attn.h"

#define GLA_CHECK_HIP(expr, code)                                                                   \
    do {                                                                                            \
        hipError_t _e = (expr);                                                                     \
        if (_e != hipSuccess) return gla::set_error((code), "%s: %s", #expr, hipGetErrorString(_e)); \
    } while (0)

namespace gla {

int set_error(int code, const char *fmt, ...);
void clear_error();

// Byte strides of a KV layout. Element (page, head, slot, i) of K sits at
//   k + page * page_stride + head * head_stride + slot * row_stride + i * esize
// and its Q8_0 scale (block i / 32) at
//   ks + page * page_stride + head * head_stride + slot * srow_stride + (i / 32) * 2.
struct KvLayout {
    const uint8_t *k;
    const uint8_t *v;
    const uint8_t *ks;
    const uint8_t *vs;
    int64_t page_stride;
    int64_t head_stride;
    int32_t row_stride;
    int32_t srow_stride;
};

// How a (batch row b, logical page lp) becomes a physical page:
//   page_table ? page_table[b * pt_stride + lp]
//              : (seq_slot ? seq_slot[b] : b) * seq_page_stride + layer_page_off + lp
//
// The device clamps every index it derives from caller data (positions to
// [0, pos_limit), sequence slots to [0, n_slots), page ids to [0, n_pages))
// so a malformed table or length reads wrong data instead of faulting.
struct PageMap {
    const int32_t *page_table;
    const int32_t *seq_slot;
    int64_t seq_page_stride;
    int64_t layer_page_off;
    int64_t n_pages;
    int32_t pt_stride;
    int32_t pos_limit;
    int32_t n_slots;
};

// Byte offset of quant K[slot][d] / V[slot][d] inside a (page, head) Q8_0
// quant block of head_dim D (16*D bytes).
__host__ __device__ __forceinline__ int q8k_off(int slot, int d, int D) {
    (void)D;
    return (d >> 6) * 1024 + (((d >> 3) & 3) * 16 + slot) * 16 + ((d >> 5) & 1) * 8 + (d & 7);
}
__host__ __device__ __forceinline__ int q8v_off(int slot, int d, int D) {
    (void)D;
    return (d >> 6) * 1024 + ((slot >> 2) * 16 + (d & 15)) * 16 + ((d >> 4) & 3) * 4 + (slot & 3);
}
// f16 index of the K scale of (slot, block) inside a (page, head) Ks array.
__host__ __device__ __forceinline__ int q8ks_off(int slot, int blk, int D) {
    return ((blk & 1) * 16 + slot) * (D >> 6) + (blk >> 1);
}

// Agent-scope (all XCDs) accesses of partials that the last workgroup to
// arrive merges inside one kernel: they bypass the per-XCD L2s, which are
// not coherent with each other within a kernel.
__device__ __forceinline__ void store_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until every memory access this thread issued has completed (its
// agent-scope stores have reached the memory all XCDs share).
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// One thread of the workgroup counts its arrival at counter *c once every
// thread's stores have completed; true in every thread of the workgroup that
// arrives last of n (which resets the counter to 0 for the next call).
__device__ __forceinline__ bool arrive_last(int32_t *c, int n, int *lds_flag) {
    wait_vm_all();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int before = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = before == n - 1;
        if (last) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *lds_flag = last;
    }
    __syncthreads();
    return *lds_flag != 0;
}

__device__ __forceinline__ int64_t map_page(const PageMap &pm, int b, int lp) {
    int64_t id;
    if (pm.page_table) {
        id = (int64_t)pm.page_table[(int64_t)b * pm.pt_stride + lp];
    } else {
        int64_t s = pm.seq_slot ? (int64_t)pm.seq_slot[b] : (int64_t)b;
        s = s < 0 ? 0 : (s >= pm.n_slots ? pm.n_slots - 1 : s);
        id = s * pm.seq_page_stride + pm.layer_page_off + lp;
    }
    return id < 0 ? 0 : (id >= pm.n_pages ? pm.n_pages - 1 : id);
}

}  // namespace gla

struct gla_ctx {
    int device = 0;
    int n_cu = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // Device scratch (decode partials, bf16 tile images, matvec pieces), one
    // buffer per stream the context has launched work on: work queued on two
    // streams at once never shares a buffer.
    struct StreamScratch {
        hipStream_t stream;
        void *ptr;
        size_t bytes;
        // arrival counters of the in-kernel merges (f32 decode, Q8_0 matvec
        // K slices): zeroed when allocated, and every call leaves them at zero
        int32_t *arrivals = nullptr;
        size_t n_arrivals = 0;
    };
    std::vector<StreamScratch> scratch;
    // device and pinned host staging of the host-pointer entry points
    void *dstage = nullptr;
    size_t dstage_bytes = 0;
    void *hstage = nullptr;
    size_t hstage_bytes = 0;
    // Buffers replaced by a larger one, kept until gla_destroy: work already
    // queued, and any HIP graph captured from the stream, still address them
    // (second: pinned host memory).
    std::vector<std::pair<void *, bool>> retired;
    // KV storages and weights created on this context: gla_destroy frees
    // their device memory and detaches the handles, so a handle released
    // after its context frees only itself.
    std::vector<gla_kv *> kvs;
    std::vector<gla_q8w *> q8ws;
    // RoPE inverse frequencies 1 / powf(base, 2p / head_dim) of the last
    // (base, head_dim) rotated on this context, computed on the host
    float rope_base = 0.0f;
    int rope_head_dim = 0;
    std::vector<float> rope_freq;
};

struct gla_kv {
    gla_ctx *ctx = nullptr;
    bool is_pool = false;
    gla_kv_dtype dtype = GLA_KV_F32;
    int n_kv_heads = 0;
    int head_dim = 0;
    int kv_dim = 0;
    // contiguous caches
    int n_seqs = 0;
    int n_layers = 0;
    int max_seq = 0;
    int pages_per_layer = 0;
    int64_t n_pages = 0;
    int64_t head_bytes = 0;
    int64_t page_bytes = 0;
    uint8_t *base = nullptr;
};

namespace gla {

KvLayout layout_of(const gla_kv *kv);
// At least `bytes` of device scratch for work on ctx->stream (grown by
// doubling; a replaced buffer stays allocated until gla_destroy).
int ensure_scratch(gla_ctx *ctx, size_t bytes, void **out);
int ensure_dstage(gla_ctx *ctx, size_t bytes);
// Free a weight handle's device memory and detach it from its context.
void detach_q8w(gla_q8w *w);
int ensure_hstage(gla_ctx *ctx, size_t bytes);

// Pages the window of one sequence spans, with the decode kernels' clamping
// of its start and length (their seq_range), from the host copies.
inline int host_seq_pages(int start, int len, int max_len, int pos_limit) {
    start = start < 0 ? 0 : start;
    len = len < 0 ? 0 : (len > max_len ? max_len : len);
    int64_t e = (int64_t)start + len;
    if (e > pos_limit) e = pos_limit;
    const int64_t s = start > e ? e : start;
    return e > s ? (int)(((e - 1) >> 4) - (s >> 4) + 1) : 0;
}

// Launchers (return GLA_OK or an error code with the message set).
struct DecodeLaunch {
    KvLayout kv;
    bool q8;
    int head_dim;
    int n_kv_heads;
    PageMap pm;
    int n_seqs;
    const int32_t *kv_start;
    const int32_t *kv_len;
    int max_kv_len;
    int n_heads;
    float scale;
    float softcap;
    const float *q;
    float *out;
    const int32_t *kv_start_host = nullptr;  // optional host copies (both or neither)
    const int32_t *kv_len_host = nullptr;
    // A caller-provided scratch buffer of scratch_cap bytes: when set the
    // launch allocates nothing and fails with GLA_ERR_INVALID if the
    // partials need more; when NULL the context's scratch is used.
    void *scratch = nullptr;
    size_t scratch_cap = 0;
    // with `scratch`: a fixed array of arrivals_cap arrival counters (zero
    // between calls), else the context's counters for its current stream
    int32_t *arrivals = nullptr;
    size_t arrivals_cap = 0;
};
// Device scratch of a decode launch: d.scratch (no allocation) or the
// context's buffer for its current stream.
int decode_scratch(gla_ctx *ctx, const DecodeLaunch &d, size_t bytes, void **out);
// At least n zeroed arrival counters for a decode launch (d.arrivals, or the
// context's for its current stream).
int decode_arrivals(gla_ctx *ctx, const DecodeLaunch &d, size_t n, int32_t **out);
// At least n zeroed arrival counters of the context for its current stream
// (every kernel that counts arrivals leaves them at zero; kernels on one
// stream run one after another, so they can share them).
int ensure_arrivals(gla_ctx *ctx, size_t n, int32_t **out);
int launch_decode(gla_ctx *ctx, const DecodeLaunch &d);
int launch_decode_q8(gla_ctx *ctx, const DecodeLaunch &d);

struct PrefillLaunch {
    KvLayout kv;
    bool q8;
    int head_dim;
    int n_kv_heads;
    PageMap pm;
    int n_seqs;
    const int32_t *q_start;
    const int32_t *pos_offset;
    int max_q_len;
    int n_heads;
    float scale;
    float softcap;
    int sliding_window;
    gla_precision precision;
    const float *q;
    float *out;
};
int launch_prefill(gla_ctx *ctx, const PrefillLaunch &p);

int launch_write_rows(gla_ctx *ctx, gla_kv *kv, const int64_t *rows, const float *k, const float *v, int n);
int launch_export_rows(gla_ctx *ctx, const gla_kv *kv, const int64_t *rows, int n, uint8_t *k_out,
                       uint8_t *v_out);
int launch_import_rows(gla_ctx *ctx, gla_kv *kv, const int64_t *rows, int n, const uint8_t *k_in,
                       const uint8_t *v_in);
int launch_copy_page(gla_ctx *ctx, gla_kv *kv, int64_t src, int64_t dst);
int launch_zero_pages(gla_ctx *ctx, gla_kv *kv, int64_t first, int64_t count);

}  // namespace gla
