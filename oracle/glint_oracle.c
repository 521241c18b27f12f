/*
 * glint_oracle.c -- TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline).
 *
 * A CPU restatement of Glint's CPU flash-attention path, in the reference's
 * loop order, so the HIP kernels can be checked against it on identical
 * inputs. Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of
 * bench.py may load this library; the product path never does.
 *
 * Restated from (all paths under the Glint repository):
 *   src/tensor/flash.rs:46-124         flash_attn_1d_ext (blocks of 32, online softmax)
 *   src/tensor/flash.rs:148-178        standard three-phase attention (test oracle)
 *   src/transformer/forward.rs:240-270 attn_heads_cpu (serial over q-heads, kv_h = h / G)
 *   src/transformer/forward.rs:574-582 window_start / attend_len rule
 *   src/transformer/forward.rs:927-958 prefill loop (parallel over query positions)
 *   src/transformer/forward.rs:1468-1502 batched decode (parallel over sequences)
 *   src/cache/mod.rs:154-164           KvCache row addressing
 *   src/cache/mod.rs:296-334           KvCacheQ8 quantize_into / dequant_range
 *   src/cache/paged.rs:453-465         PagedKvCache read: table[layer][pos/16], slot pos%16
 *   src/tensor/ops.rs:212-245          rope (adjacent pairs, partial rot_dim, linear scaling)
 *   src/tensor/quantized.rs:587-610    matvec_q8_0_scalar (per-block i8 x f32 sums, then x scale)
 *   half 2.7.1 f16::from_f32 / to_f32  (third-party; restated as IEEE round-to-nearest-even)
 *
 * Build flags (oracle/Makefile): -O2 -ffp-contract=off, no fast-math, so the
 * float operations happen in the same order and rounding as the scalar Rust
 * (Rust never contracts a*b+c into an FMA). expf/tanhf come from glibc, as
 * Rust's f32::exp/f32::tanh do on Linux.
 *
 * Parity status of each function is recorded in the tests that pin it
 * (tests/test_oracle.py). Unpinned at bit level: agreement with the compiled
 * Rust binary itself (rustc is not available); every value-level property is
 * pinned by the reference's fixtures, closed forms and an f64 brute force.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_BLOCK 32  /* src/tensor/flash.rs:10 BLOCK_SIZE */
#define OR_PAGE 16   /* src/cache/paged.rs:55 PAGE_SIZE */
#define OR_MAXD 1024 /* largest head_dim the oracle's stack buffers hold */

/* Planted mistakes for the tests that show each pin catches a plausible bug
 * (tests/test_oracle.py builds with -DOR_MUTANT=n; the default build has none):
 *   1 drop the rescale of `out`     2 GQA head map h % G      3 window off by one
 *   4 f16 narrowing truncates       5 quantise rounds to even 6 paged slot index shifted
 *   7 soft-cap without the divide   8 f16 scale read big-endian
 *   9 prefill excludes its own position                       10 scale applied twice */
#ifndef OR_MUTANT
#define OR_MUTANT 0
#endif

/* ---------------------------------------------------------------------------
 * f16 <-> f32 (half 2.7.1, used at src/cache/mod.rs:306 and :325).
 * IEEE 754 binary16, round-to-nearest-even on narrowing.
 * ------------------------------------------------------------------------- */
uint16_t or_f16_from_f32(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e32 = (int)(ax >> 23);
    int e = e32 - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e >= 1) {
        uint32_t h = ((uint32_t)e << 10) | ((ax & 0x7fffffu) >> 13);
        uint32_t rem = ax & 0x1fffu;
        if (OR_MUTANT == 4) rem = 0;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may reach inf: correct */
        return (uint16_t)(sign | h);
    }
    /* subnormal or zero in f16: value = h * 2^-24 */
    if (e32 == 0) return (uint16_t)sign; /* f32 subnormals are far below 2^-25 */
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    int shift = 126 - e32; /* >= 14 */
    if (shift > 24) return (uint16_t)sign;
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24, exact in f32 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ---------------------------------------------------------------------------
 * Q8_0 row codec -- src/cache/mod.rs:296-334.
 * Row = ceil(n/32) blocks of [f16 d little-endian][32 x i8] = 34 bytes.
 * ------------------------------------------------------------------------- */
void or_q8_quantize_row(const float *src, int n, uint8_t *dst) {
    int n_blocks = (n + 31) / 32;
    for (int b = 0; b < n_blocks; b++) {
        int start = b * 32;
        int end = start + 32 < n ? start + 32 : n;
        float max_abs = 0.0f; /* fold(0.0, f32::max): NaN elements are skipped */
        for (int j = start; j < end; j++) max_abs = fmaxf(max_abs, fabsf(src[j]));
        float d = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
        float inv_d = 1.0f / d;
        uint8_t *out = dst + (size_t)b * 34;
        uint16_t hd = or_f16_from_f32(d);
        out[0] = (uint8_t)(hd & 0xff);
        out[1] = (uint8_t)(hd >> 8);
        for (int j = start; j < end; j++) {
            float r = roundf(src[j] * inv_d); /* round half away from zero, like f32::round */
            if (OR_MUTANT == 5) r = rintf(src[j] * inv_d);
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            int8_t qv = isnan(r) ? 0 : (int8_t)r; /* Rust `as i8` maps NaN to 0 */
            out[2 + (j - start)] = (uint8_t)qv;
        }
        for (int j = end - start; j < 32; j++) out[2 + j] = 0;
    }
}

void or_q8_dequant_range(const uint8_t *row, int start_elem, int end_elem, float *buf) {
    int first_block = start_elem / 32;
    int last_block = (end_elem - 1) / 32;
    int out_idx = 0;
    for (int b = first_block; b <= last_block; b++) {
        const uint8_t *block = row + (size_t)b * 34;
        float d = or_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
        if (OR_MUTANT == 8) d = or_f16_to_f32((uint16_t)(block[1] | (block[0] << 8)));
        for (int j = 0; j < 32; j++) {
            int elem = b * 32 + j;
            if (elem >= start_elem && elem < end_elem) {
                buf[out_idx++] = (float)(int8_t)block[2 + j] * d;
            }
        }
    }
}

/* ---------------------------------------------------------------------------
 * KV stores -- the KvStore implementations on the path (src/cache/mod.rs:24-109).
 * ------------------------------------------------------------------------- */
enum { OR_F32 = 0, OR_Q8 = 1, OR_PAGED_F32 = 2, OR_PAGED_Q8 = 3 };

typedef struct or_store {
    int kind;
    int n_layers;
    int max_seq;       /* contiguous kinds: rows per layer */
    int kv_dim;        /* n_kv_heads * head_dim */
    int bytes_per_pos; /* Q8 kinds: ceil(kv_dim / 32) * 34 */
    const float *kf, *vf;   /* F32: [layer][max_seq][kv_dim]; PAGED_F32: [page][16][kv_dim] */
    const uint8_t *kq, *vq; /* Q8: [layer][max_seq][bpp];    PAGED_Q8: [page][16][bpp] */
    const int32_t *table;   /* paged kinds: table[layer * table_stride + logical_page] */
    int table_stride;
} or_store;

or_store *or_store_new(int kind, int n_layers, int max_seq, int kv_dim, const void *k, const void *v,
                       const int32_t *table, int table_stride) {
    or_store *s = (or_store *)calloc(1, sizeof(or_store));
    s->kind = kind;
    s->n_layers = n_layers;
    s->max_seq = max_seq;
    s->kv_dim = kv_dim;
    s->bytes_per_pos = ((kv_dim + 31) / 32) * 34;
    if (kind == OR_F32 || kind == OR_PAGED_F32) {
        s->kf = (const float *)k;
        s->vf = (const float *)v;
    } else {
        s->kq = (const uint8_t *)k;
        s->vq = (const uint8_t *)v;
    }
    s->table = table;
    s->table_stride = table_stride;
    return s;
}

void or_store_free(or_store *s) { free(s); }

/* read_k_head / read_v_head: src/cache/mod.rs:154-164 (f32), :336-358 (Q8),
 * src/cache/paged.rs:453-465 (paged). which: 0 = K, 1 = V. */
static void or_read_head(const or_store *s, int which, int layer, long pos, int kv_h, int d, float *buf) {
    switch (s->kind) {
    case OR_F32: {
        const float *base = which ? s->vf : s->kf;
        size_t start = ((size_t)layer * s->max_seq + pos) * s->kv_dim + (size_t)kv_h * d;
        memcpy(buf, base + start, sizeof(float) * d);
        break;
    }
    case OR_Q8: {
        const uint8_t *base = which ? s->vq : s->kq;
        const uint8_t *row = base + ((size_t)layer * s->max_seq + pos) * s->bytes_per_pos;
        or_q8_dequant_range(row, kv_h * d, (kv_h + 1) * d, buf);
        break;
    }
    case OR_PAGED_F32: {
        const float *base = which ? s->vf : s->kf;
        int32_t page = s->table[(size_t)layer * s->table_stride + pos / OR_PAGE];
        size_t start = ((size_t)page * OR_PAGE + (OR_MUTANT == 6 ? (pos + 1) : pos) % OR_PAGE) * s->kv_dim +
                       (size_t)kv_h * d;
        memcpy(buf, base + start, sizeof(float) * d);
        break;
    }
    default: { /* OR_PAGED_Q8: paged indexing in front of the Q8 row codec */
        const uint8_t *base = which ? s->vq : s->kq;
        int32_t page = s->table[(size_t)layer * s->table_stride + pos / OR_PAGE];
        const uint8_t *row = base + ((size_t)page * OR_PAGE + pos % OR_PAGE) * s->bytes_per_pos;
        or_q8_dequant_range(row, kv_h * d, (kv_h + 1) * d, buf);
        break;
    }
    }
}

void or_read_k_head(const or_store *s, int layer, long pos, int kv_h, int d, float *buf) {
    or_read_head(s, 0, layer, pos, kv_h, d, buf);
}
void or_read_v_head(const or_store *s, int layer, long pos, int kv_h, int d, float *buf) {
    or_read_head(s, 1, layer, pos, kv_h, d, buf);
}

/* ---------------------------------------------------------------------------
 * flash_attn_1d_ext -- src/tensor/flash.rs:46-124. `out` must be pre-zeroed.
 * has_cap = 0 means softcap None.
 * ------------------------------------------------------------------------- */
void or_flash_attn_1d_ext(const float *q, const or_store *cache, int layer, int kv_h, long start_pos,
                          long seq_len, int head_dim, float scale, int has_cap, float cap, float *out) {
    float k_buf[OR_MAXD];
    float v_buf[OR_MAXD];
    float m = -INFINITY;
    float l = 0.0f;
    long start = 0;
    while (start < seq_len) {
        long end = start + OR_BLOCK < seq_len ? start + OR_BLOCK : seq_len;
        int block_len = (int)(end - start);
        float scores[OR_BLOCK] = {0};

        /* Phase 1 -- Q . K scores (flash.rs:75-88) */
        for (int i = 0; i < block_len; i++) {
            or_read_head(cache, 0, layer, start_pos + start + i, kv_h, head_dim, k_buf);
            float dot = 0.0f;
            for (int d = 0; d < head_dim; d++) dot += q[d] * k_buf[d];
            float s = dot * scale;
            if (OR_MUTANT == 10) s *= scale;
            if (has_cap) s = (OR_MUTANT == 7) ? cap * tanhf(s) : cap * tanhf(s / cap);
            scores[i] = s;
        }

        /* Phase 2 -- running maximum and rescale (flash.rs:90-103) */
        float m_block = -INFINITY;
        for (int i = 0; i < block_len; i++)
            if (scores[i] > m_block) m_block = scores[i];
        float m_new = fmaxf(m, m_block);
        float rescale = expf(m - m_new);
        if (OR_MUTANT != 1)
            for (int d = 0; d < head_dim; d++) out[d] *= rescale;
        l *= rescale;

        /* Phase 3 -- V accumulation (flash.rs:105-113) */
        for (int i = 0; i < block_len; i++) {
            float e = expf(scores[i] - m_new);
            or_read_head(cache, 1, layer, start_pos + start + i, kv_h, head_dim, v_buf);
            for (int d = 0; d < head_dim; d++) out[d] += e * v_buf[d];
            l += e;
        }
        m = m_new;
        start = end;
    }
    if (l > 0.0f) { /* flash.rs:118-123 */
        float inv_l = 1.0f / l;
        for (int d = 0; d < head_dim; d++) out[d] *= inv_l;
    }
}

/* ---------------------------------------------------------------------------
 * Standard three-phase attention -- src/tensor/flash.rs:148-178, with the
 * soft-cap placement of the uncached path src/transformer/forward.rs:209-214
 * and softmax of src/tensor/ops.rs:183-192. Writes (not accumulates) `out`.
 * ------------------------------------------------------------------------- */
void or_standard_attn(const float *q, const or_store *cache, int layer, int kv_h, long start_pos,
                      long seq_len, int head_dim, float scale, int has_cap, float cap, float *out) {
    float *scores = (float *)malloc(sizeof(float) * (seq_len > 0 ? seq_len : 1));
    float k_buf[OR_MAXD];
    float v_buf[OR_MAXD];
    for (long s = 0; s < seq_len; s++) {
        or_read_head(cache, 0, layer, start_pos + s, kv_h, head_dim, k_buf);
        float dot = 0.0f;
        for (int d = 0; d < head_dim; d++) dot += q[d] * k_buf[d];
        float sc = dot * scale;
        if (has_cap) sc = cap * tanhf(sc / cap);
        scores[s] = sc;
    }
    float max_s = -INFINITY;
    for (long s = 0; s < seq_len; s++) max_s = fmaxf(max_s, scores[s]);
    float sum = 0.0f;
    for (long s = 0; s < seq_len; s++) {
        scores[s] = expf(scores[s] - max_s);
        sum += scores[s];
    }
    for (int d = 0; d < head_dim; d++) out[d] = 0.0f;
    for (long s = 0; s < seq_len; s++) {
        float w = scores[s] / sum;
        or_read_head(cache, 1, layer, start_pos + s, kv_h, head_dim, v_buf);
        for (int d = 0; d < head_dim; d++) out[d] += w * v_buf[d];
    }
    free(scores);
}

/* ---------------------------------------------------------------------------
 * attn_heads_cpu -- src/transformer/forward.rs:240-270. `out` pre-zeroed.
 * ------------------------------------------------------------------------- */
void or_attn_heads_cpu(const float *q_all, const or_store *cache, int layer, long window_start,
                       long attend_len, int n_heads, int kv_group_size, int head_dim, float scale,
                       int has_cap, float cap, float *out) {
    for (int h = 0; h < n_heads; h++) {
        int kv_h = (OR_MUTANT == 2) ? h % kv_group_size : h / kv_group_size;
        size_t off = (size_t)h * head_dim;
        or_flash_attn_1d_ext(q_all + off, cache, layer, kv_h, window_start, attend_len, head_dim, scale,
                             has_cap, cap, out + off);
    }
}

/* window_start rule -- src/transformer/forward.rs:574-581 (decode), :884-893
 * (prefill), :1474-1483 (batch). sliding_window <= 0 means None. */
long or_window_start(long pos, long sliding_window, int alternating, int layer) {
    if (alternating && (layer % 2) != 0) return 0;
    if (sliding_window <= 0) return 0;
    long w = pos - sliding_window + (OR_MUTANT == 3 ? 0 : 1);
    return w > 0 ? w : 0;
}

/* ---------------------------------------------------------------------------
 * Parallel-for over independent tasks (the Rayon into_par_iter split; each
 * task has one writer, so scheduling has no numerical effect).
 * ------------------------------------------------------------------------- */
typedef struct {
    void (*fn)(void *, long);
    void *arg;
    long n;
    long next;
} or_pfor;

static void *or_pfor_worker(void *p) {
    or_pfor *pf = (or_pfor *)p;
    for (;;) {
        long i = __atomic_fetch_add(&pf->next, 1, __ATOMIC_RELAXED);
        if (i >= pf->n) break;
        pf->fn(pf->arg, i);
    }
    return NULL;
}

static void or_parallel_for(long n, int n_threads, void (*fn)(void *, long), void *arg) {
    or_pfor pf = {fn, arg, n, 0};
    if (n_threads <= 1 || n <= 1) {
        or_pfor_worker(&pf);
        return;
    }
    if (n_threads > 256) n_threads = 256;
    pthread_t th[256];
    int started = 0;
    for (int t = 1; t < n_threads; t++)
        if (pthread_create(&th[started], NULL, or_pfor_worker, &pf) == 0) started++;
    or_pfor_worker(&pf);
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
}

/* ---------------------------------------------------------------------------
 * Batched decode attention -- src/transformer/forward.rs:1468-1502: one task
 * per sequence, each running attn_heads_cpu over its own cache and window.
 * kv_start / kv_len are the per-sequence window_start / attend_len.
 * ------------------------------------------------------------------------- */
typedef struct {
    const float *q;
    const or_store *const *caches;
    int layer;
    const long *kv_start;
    const long *kv_len;
    int n_heads, n_kv_heads, head_dim;
    float scale;
    int has_cap;
    float cap;
    float *out;
} or_batch_args;

static void or_batch_task(void *p, long s) {
    const or_batch_args *a = (const or_batch_args *)p;
    size_t q_dim = (size_t)a->n_heads * a->head_dim;
    float *o = a->out + s * q_dim;
    memset(o, 0, sizeof(float) * q_dim);
    or_attn_heads_cpu(a->q + s * q_dim, a->caches[s], a->layer, a->kv_start[s], a->kv_len[s], a->n_heads,
                      a->n_heads / a->n_kv_heads, a->head_dim, a->scale, a->has_cap, a->cap, o);
}

void or_decode_batch(const float *q, const or_store *const *caches, int n_seqs, int layer,
                     const long *kv_start, const long *kv_len, int n_heads, int n_kv_heads, int head_dim,
                     float scale, int has_cap, float cap, float *out, int n_threads) {
    or_batch_args a = {q, caches, layer, kv_start, kv_len, n_heads, n_kv_heads, head_dim, scale,
                       has_cap, cap, out};
    or_parallel_for(n_seqs, n_threads, or_batch_task, &a);
}

/* ---------------------------------------------------------------------------
 * Prefill attention -- src/transformer/forward.rs:927-958: one task per query
 * position lp; abs = pos_offset + lp; window per the rule above; every head
 * runs flash_attn_1d_ext over [window, abs].
 * q, out: [seq_len][n_heads * head_dim].
 * ------------------------------------------------------------------------- */
typedef struct {
    const float *q;
    const or_store *cache;
    int layer;
    long pos_offset;
    int n_heads, n_kv_heads, head_dim;
    float scale;
    int has_cap;
    float cap;
    long sliding_window;
    int alternating;
    float *out;
} or_prefill_args;

static void or_prefill_task(void *p, long lp) {
    const or_prefill_args *a = (const or_prefill_args *)p;
    size_t q_dim = (size_t)a->n_heads * a->head_dim;
    long abs_pos = a->pos_offset + lp;
    long window = or_window_start(abs_pos, a->sliding_window, a->alternating, a->layer);
    long attend_len = abs_pos + (OR_MUTANT == 9 ? 0 : 1) - window;
    float *o = a->out + lp * q_dim;
    memset(o, 0, sizeof(float) * q_dim);
    int group = a->n_heads / a->n_kv_heads;
    for (int h = 0; h < a->n_heads; h++) {
        size_t off = (size_t)h * a->head_dim;
        int kv_h = (OR_MUTANT == 2) ? h % group : h / group;
        or_flash_attn_1d_ext(a->q + lp * q_dim + off, a->cache, a->layer, kv_h, window, attend_len,
                             a->head_dim, a->scale, a->has_cap, a->cap, o + off);
    }
}

void or_prefill(const float *q, const or_store *cache, int layer, long pos_offset, long seq_len, int n_heads,
                int n_kv_heads, int head_dim, float scale, int has_cap, float cap, long sliding_window,
                int alternating, float *out, int n_threads) {
    or_prefill_args a = {q, cache, layer, pos_offset, n_heads, n_kv_heads, head_dim, scale, has_cap, cap,
                         sliding_window, alternating, out};
    or_parallel_for(seq_len, n_threads, or_prefill_task, &a);
}

/* Parallel Q8 quantisation of many rows (the KvStore::write codec applied
 * row by row, src/cache/mod.rs:386-387); used to build paged-Q8 fixtures. */
typedef struct {
    const float *src;
    uint8_t *dst;
    int n;
    int bpp;
} or_qrows_args;

static void or_qrows_task(void *p, long r) {
    const or_qrows_args *a = (const or_qrows_args *)p;
    or_q8_quantize_row(a->src + (size_t)r * a->n, a->n, a->dst + (size_t)r * a->bpp);
}

void or_q8_quantize_rows(const float *src, long n_rows, int n, uint8_t *dst, int n_threads) {
    or_qrows_args a = {src, dst, n, ((n + 31) / 32) * 34};
    or_parallel_for(n_rows, n_threads, or_qrows_task, &a);
}

/* rope, src/tensor/ops.rs:212-245: x holds whole heads of head_dim; for each
 * even i < (min(rot_dim, head_dim) & ~1), freq = 1 / base^(i / head_dim),
 * angle = (pos / scaling_factor) * freq, and every head's pair (i, i+1) is
 * rotated by angle; the other dimensions are copied. */
void or_rope(const float *x, float *out, int n, long pos, int head_dim, float freq_base, float scaling_factor,
             int rot_dim) {
    memcpy(out, x, (size_t)n * sizeof(float));
    const float pos_scaled = (float)pos / scaling_factor;
    const int rot = (rot_dim < head_dim ? rot_dim : head_dim) & ~1;
    for (int i = 0; i < rot; i += 2) {
        const float freq = 1.0f / powf(freq_base, (float)i / (float)head_dim);
        const float angle = pos_scaled * freq;
        const float c = cosf(angle);
        const float s = sinf(angle);
        for (int off = 0; off + head_dim <= n; off += head_dim) {
            const float x0 = x[off + i];
            const float x1 = x[off + i + 1];
            out[off + i] = x0 * c - x1 * s;
            out[off + i + 1] = x0 * s + x1 * c;
        }
    }
}

/* matvec_q8_0_scalar, src/tensor/quantized.rs:587-610: rows of cols/32
 * GGML Q8_0 blocks ([f16 scale LE][32 x i8], 34 bytes); out[i] = sum over
 * blocks of (sum_j i8 * vec[j] in f32, in order) * scale. */
void or_matvec_q8_0(const uint8_t *data, long rows, int cols, const float *vec, float *out) {
    const int n_blocks = cols / 32;
    const size_t bytes_per_row = (size_t)n_blocks * 34;
    for (long i = 0; i < rows; i++) {
        const uint8_t *row = data + (size_t)i * bytes_per_row;
        float sum = 0.0f;
        for (int b = 0; b < n_blocks; b++) {
            const uint8_t *block = row + (size_t)b * 34;
            const float scale = or_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
            float block_sum = 0.0f;
            for (int j = 0; j < 32; j++) block_sum += (float)(int8_t)block[2 + j] * vec[b * 32 + j];
            sum += block_sum * scale;
        }
        out[i] = sum;
    }
}
