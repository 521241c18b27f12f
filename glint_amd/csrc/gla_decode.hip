// gla_decode.hip -- single-token decode attention for gfx950 (HBM-bound).
//
// Math: flash_attn_1d_ext (src/tensor/flash.rs:46-124) for every q-head of a
// batch, as attn_heads_cpu runs it (src/transformer/forward.rs:240-270).
//
// Work decomposition (split-K / flash-decoding):
//   grid = (kv_head x head_group, split, sequence), 256 threads (4 waves).
//   A workgroup owns `pps` consecutive pages of one sequence and one KV head,
//   and all GT q-heads that read that KV head (GQA: K/V are read once for the
//   whole group). Each wave takes whole pages; inside a wave 8 lanes share a
//   token row (each lane owns D/8 elements, loaded as 16-byte chunks so 8
//   lanes cover 128 contiguous bytes) and the 8 lane groups take 8 different
//   tokens. A lane group keeps its own online-softmax state (m, l, acc) in
//   the log2 domain; the groups are merged with shuffles once per split, the
//   4 waves through LDS, and splits by decode_combine_kernel.
// Batch invariance: `pps` is a function of the sequence's own window
// (split_pages), so where its splits fall, and with them every rounding of
// its result, is the same whatever else is in the batch -- the reference's
// batched == single guarantee (src/transformer/forward.rs:1946-2002).
// This file serves f32 storage; Q8_0 storage has its own MFMA kernel
// (gla_decode_q8.hip).
#include <float.h>
#include <math.h>
#include <stdlib.h>

#include <algorithm>

#include "gla_internal.h"

namespace gla {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kStepsPerIter = 2;  // half-page token steps a lane group loads per iteration
// A window of few splits merges them in the last of its workgroups to finish
// instead of a combine launch. That workgroup's threads each merge
// EPT = ceil(GT x D / 256) elements, reading their splits' partials in
// batches of eight splits, one memory round trip per batch; the merge pays
// for up to two batches, 16 splits of 4 pages. The bound is in pages and adds
// the page a start inside a page brings (65 pages, a third batch of one
// split), so a launch sized from max_kv_len = 1024 without host lengths needs
// no combine. Above 2 elements per thread (a batch is 24 x EPT loads in flight
// per thread) the bound is one batch, 33 pages.
constexpr int merge_ept(int D, int gt) { return (gt * D + kThreads - 1) / kThreads; }
constexpr int merge_max_pages(int D, int gt) { return merge_ept(D, gt) <= 2 ? 65 : 33; }

struct DecodeParams {
    KvLayout kv;
    PageMap pm;
    const int32_t *kv_start;
    const int32_t *kv_len;
    const float *q;
    float *out;
    float *part_acc;  // [unit][split][GT][D]
    float *part_ml;   // [unit][split] one 128-byte line: m[GT] at 0, l[GT] at 8, zeros
    int n_heads;
    int n_kv_heads;
    int group;  // n_heads / n_kv_heads
    int n_hg;   // head groups per kv head
    int pps_fixed;  // pages per split for every window (tuning override), or 0: split_pages
    int max_splits;
    int max_len;  // host bound on kv_len: lengths are clamped to it, so splits never exceed max_splits
    float q_mul;    // multiplier of q.k: scale*log2(e), or scale with a soft-cap
    float softcap;  // > 0: cap * tanh(s / cap)
    // Windows of more than one split and at most merge_pages pages are merged
    // by the last of their workgroups to finish, counted in arrivals[unit] (0
    // between calls: the last arrival resets it); longer windows by
    // decode_combine_kernel.
    int merge_pages;
    int32_t *arrivals;
};

// Sum over the 8 lanes of an aligned lane group (DPP: quad xor1, quad xor2,
// half-row mirror).
__device__ __forceinline__ float sum8(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// x combined with lane ^ 8 / ^ 16 / ^ 32 on the VALU (DPP row rotation and the
// gfx950 row swaps), no LDS round trip: the merge of the 8 lane groups.
__device__ __forceinline__ float other8(float x) {  // lane ^ 8 within a row of 16
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
}
__device__ __forceinline__ float add16(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ __forceinline__ float add32(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ __forceinline__ float max16(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
__device__ __forceinline__ float max32(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
// Two values' row-pair sums with one swap: rows 0 and 2 of the result hold
// x's r0 + r1 and r2 + r3, rows 1 and 3 y's (v_permlane16_swap exchanges
// rows 1, 3 of x with rows 0, 2 of y).
__device__ __forceinline__ float pair16(float x, float y) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
// Two pair16 results s (of x, y) and t (of z, w) summed across the halves:
// row 0 holds x's total, row 1 y's, row 2 z's, row 3 w's.
__device__ __forceinline__ float pair32(float s, float t) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(t), false, false);
    return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}

// tanh(x) = sign(x) (1 - t) / (1 + t), t = exp(-2|x|).
__device__ __forceinline__ float tanh_approx(float x) {
    float t = fast_exp2(-2.0f * kLog2e * fabsf(x));
    float r = (1.0f - t) / (1.0f + t);
    return copysignf(r, x);
}

// Pages per split of a window spanning n pages: 4 up to 128 pages, 8 up to
// 256, 12 up to 384, then 16. A function of the window alone (see the file
// comment); it gives a single sequence enough splits to spread over the
// chip (cfg2, 256 pages: 32 splits of 8 measured 14.6 us per layer against
// 16.1 with 64 of 4 and 16.4 with 16 of 16; cfg1, 32 pages: 8 splits of 4
// pages, 7.6 us per call, against 8.3 with 8-page splits).
__host__ __device__ __forceinline__ int split_pages(int n_pages) {
    const int p = 4 * ((n_pages + 127) / 128);
    return p < 4 ? 4 : (p > 16 ? 16 : p);
}

// The most splits split_pages gives any window of at most n pages.
int max_splits_upto(int n) {
    if (n <= 128) return (n + 3) / 4;
    return std::max(32, (n + 15) / 16);
}

// Range of pages and splits of sequence b, after clamping to the storage.
struct SeqRange {
    int start, end;  // positions [start, end)
    int fp;          // first logical page
    int n_pages;
    int pps;         // pages per split
    int n_splits;
};

__device__ __forceinline__ SeqRange seq_range(const DecodeParams &p, int b) {
    SeqRange r;
    int s = p.kv_start[b];
    int len = p.kv_len[b];
    s = s < 0 ? 0 : s;
    len = len < 0 ? 0 : (len > p.max_len ? p.max_len : len);
    int e = s + len;
    if (e > p.pm.pos_limit) e = p.pm.pos_limit;
    if (s > e) s = e;
    r.start = s;
    r.end = e;
    if (e > s) {
        r.fp = s >> 4;
        r.n_pages = ((e - 1) >> 4) - r.fp + 1;
        r.pps = p.pps_fixed > 0 ? p.pps_fixed : split_pages(r.n_pages);
        r.n_splits = min((r.n_pages + r.pps - 1) / r.pps, p.max_splits);
    } else {
        r.fp = 0;
        r.n_pages = 0;
        r.pps = 1;
        r.n_splits = 0;
    }
    return r;
}

// 16-byte non-temporal load: K/V bytes are read once per call.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_nt(const uint8_t *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float word_f(const uint4 &c, int w) {
    return __uint_as_float(w == 0 ? c.x : (w == 1 ? c.y : (w == 2 ? c.z : c.w)));
}

// The last-arriving workgroup's merge of a short window: thread tid merges
// elements tid, tid + 256, ... (EPT of them) of the unit's gcount x D outputs,
// in split order, eight splits at a time; each batch's loads for all of the
// thread's elements are issued together (one memory round trip per batch), and
// (M, L, A) absorb a batch with one rescale.
template <int D, int GT>
__device__ __forceinline__ void merge_splits_agent(const DecodeParams &p, int64_t slot0, int n_splits, int gcount,
                                                   float *out) {
    constexpr int EPT = merge_ept(D, GT);
    const int tid = threadIdx.x;
    const int n_el = gcount * D;
    int gk[EPT], ek[EPT];
    float M[EPT], L[EPT], A[EPT];
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int idx = min(tid + k * kThreads, n_el - 1);
        gk[k] = idx / D;
        ek[k] = idx - gk[k] * D;
        M[k] = -INFINITY;
        L[k] = 0.0f;
        A[k] = 0.0f;
    }
    for (int s0 = 0; s0 < n_splits; s0 += 8) {
        float mi[EPT][8], li[EPT][8], ai[EPT][8];
#pragma unroll
        for (int k = 0; k < EPT; k++) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int64_t slot = slot0 + min(s0 + j, n_splits - 1);
                mi[k][j] = load_agent(p.part_ml + slot * 32 + gk[k]);
                li[k][j] = load_agent(p.part_ml + slot * 32 + 8 + gk[k]);
                ai[k][j] = load_agent(p.part_acc + (slot * GT + gk[k]) * D + ek[k]);
            }
        }
        const int nv = n_splits - s0;
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            float bm = M[k];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (j < nv) bm = fmaxf(bm, mi[k][j]);
            const float f0 = (M[k] == -INFINITY) ? 0.0f : fast_exp2(M[k] - bm);
            L[k] *= f0;
            A[k] *= f0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (j < nv) {
                    const float f = (mi[k][j] == -INFINITY) ? 0.0f : fast_exp2(mi[k][j] - bm);
                    L[k] = fmaf(li[k][j], f, L[k]);
                    A[k] = fmaf(ai[k][j], f, A[k]);
                }
            }
            M[k] = bm;
        }
    }
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int idx = tid + k * kThreads;
        if (idx < n_el) out[idx] = L[k] > 0.0f ? A[k] * (1.0f / L[k]) : A[k];  // (a NaN sum stays NaN, as flash.rs:118-123)
    }
}

template <int D, int GT, int NSTEP, bool CAP>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(const DecodeParams p) {
    constexpr int EPL = D / 8;       // elements per lane
    constexpr int EPC = 4;           // floats per 16-byte chunk
    constexpr int NCH = EPL / EPC;   // chunks per lane
    constexpr int PPW = NSTEP / 2;   // pages per wave per iteration

    __shared__ float lds_acc[kWaves][GT][D];
    __shared__ float lds_m[kWaves][GT];
    __shared__ float lds_l[kWaves][GT];

    // grid (KV head x head group, split, sequence): head index fastest, so
    // the head spans of the same pages are read together
    const int split = blockIdx.y;
    const int b = blockIdx.z;
    const int kvh = blockIdx.x / p.n_hg;
    const int hg = blockIdx.x - kvh * p.n_hg;
    const int g0 = hg * GT;
    const int gcount = min(GT, p.group - g0);
    const int h_base = kvh * p.group + g0;

    const SeqRange r = seq_range(p, b);
    const int tid = threadIdx.x;
    if (r.n_pages == 0) {  // empty window: zero output (the reference's pre-zeroed buffer)
        if (split == 0)
            for (int idx = tid; idx < gcount * D; idx += kThreads)
                p.out[((int64_t)b * p.n_heads + h_base) * D + idx] = 0.0f;
        return;
    }
    if (split >= r.n_splits) return;
    const int pg0 = r.fp + split * r.pps;
    // (the last split takes what is left; it only differs from pg0 + pps when
    // the device lengths exceed what max_splits was sized for)
    const int pg1 = split + 1 == r.n_splits ? r.fp + r.n_pages : min(r.fp + r.n_pages, pg0 + r.pps);

    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int tg = lane >> 3;
    const int sub = lane & 7;

    // q for the GT heads, in the lane's element order: chunk i covers
    // elements (i*8 + sub)*EPC .. +EPC.
    float qv[GT][EPL];
#pragma unroll
    for (int g = 0; g < GT; g++) {
        const int gg = g < gcount ? g : gcount - 1;
        const float *qp = p.q + ((int64_t)b * p.n_heads + h_base + gg) * D;
#pragma unroll
        for (int i = 0; i < NCH; i++) {
#pragma unroll
            for (int e = 0; e < EPC; e++) qv[g][i * EPC + e] = qp[(i * 8 + sub) * EPC + e];
        }
    }

    float m[GT], l[GT], acc[GT][EPL];
#pragma unroll
    for (int g = 0; g < GT; g++) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[g][e] = 0.0f;
    }

    const int64_t head_off = (int64_t)kvh * p.kv.head_stride;

    for (int pb = pg0 + wave * PPW; pb < pg1; pb += kWaves * PPW) {
        uint4 kr[NSTEP][NCH], vr[NSTEP][NCH];
        bool valid[NSTEP];
        int64_t pid[PPW];
#pragma unroll
        for (int j = 0; j < PPW; j++) pid[j] = map_page(p.pm, b, (pb + j < pg1) ? pb + j : pb);
#pragma unroll
        for (int s = 0; s < NSTEP; s++) {
            const int page = pb + s / 2;
            const int slot = (s & 1) * 8 + tg;
            const int pos = page * 16 + slot;
            valid[s] = page < pg1 && pos >= r.start && pos < r.end;
            const int64_t base = pid[s / 2] * p.kv.page_stride + head_off + (int64_t)slot * p.kv.row_stride;
            const uint8_t *kp = p.kv.k + base;
            const uint8_t *vp = p.kv.v + base;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
                kr[s][i] = load_nt(kp + (i * 8 + sub) * 16);
                vr[s][i] = load_nt(vp + (i * 8 + sub) * 16);
            }
        }

        // scores of the NSTEP tokens of this lane group, log2 domain
        float t[NSTEP][GT];
#pragma unroll
        for (int s = 0; s < NSTEP; s++) {
            float dot[GT];
#pragma unroll
            for (int g = 0; g < GT; g++) dot[g] = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; i++) {
#pragma unroll
                for (int e = 0; e < EPC; e++) {
                    const float kf = word_f(kr[s][i], e);
#pragma unroll
                    for (int g = 0; g < GT; g++) dot[g] = fmaf(qv[g][i * EPC + e], kf, dot[g]);
                }
            }
#pragma unroll
            for (int g = 0; g < GT; g++) {
                // q_mul on the score, not on q: q's loads then have no use
                // before the K/V loads are issued, so their wait comes after
                float x = sum8(dot[g]) * p.q_mul;
                // (a template argument: a runtime test here became a branch
                // around every score)
                if constexpr (CAP) x = p.softcap * tanh_approx(x / p.softcap) * kLog2e;
                t[s][g] = x;
            }
        }

        // running maximum; rescale only when it grows
#pragma unroll
        for (int g = 0; g < GT; g++) {
            float mx = m[g];
#pragma unroll
            for (int s = 0; s < NSTEP; s++)
                if (valid[s]) mx = fmaxf(mx, t[s][g]);
            if (mx > m[g]) {
                const float rs = fast_exp2(m[g] - mx);
                l[g] *= rs;
#pragma unroll
                for (int e = 0; e < EPL; e++) acc[g][e] *= rs;
                m[g] = mx;
            }
        }

        // P . V
#pragma unroll
        for (int s = 0; s < NSTEP; s++) {
            if (!valid[s]) {
#pragma unroll
                for (int i = 0; i < NCH; i++) vr[s][i] = make_uint4(0, 0, 0, 0);
            }
            float pw[GT];
#pragma unroll
            for (int g = 0; g < GT; g++) {
                pw[g] = valid[s] ? fast_exp2(t[s][g] - m[g]) : 0.0f;
                l[g] += pw[g];
            }
#pragma unroll
            for (int i = 0; i < NCH; i++) {
#pragma unroll
                for (int e = 0; e < EPC; e++) {
                    const float vf = word_f(vr[s][i], e);
#pragma unroll
                    for (int g = 0; g < GT; g++) acc[g][i * EPC + e] = fmaf(pw[g], vf, acc[g][i * EPC + e]);
                }
            }
        }
    }

    // merge the 8 lane groups of the wave (lanes with equal `sub` own the
    // same elements): the maxima and sums of each head as all-reductions,
    // the GT x EPL output sums as a reduce-scatter over the same tree
    // (lane ^ 8, then ^ 16, then ^ 32) with two values per row swap: after
    // it, row r of the wave holds value 4k + r of each group of four, and
    // the row's first 8 lanes write it. The first step is written as the
    // fused multiply-add it compiles to, so that every value rounds alike
    // (left to the compiler, the contraction differs between values).
#pragma unroll
    for (int g = 0; g < GT; g++) {
        float M = m[g];
        M = max32(max16(fmaxf(M, other8(M))));
        const float f = (m[g] == -INFINITY) ? 0.0f : fast_exp2(m[g] - M);
        float lg = fmaf(l[g], f, other8(l[g] * f));
        lg = add32(add16(lg));
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[g][e] = fmaf(acc[g][e], f, other8(acc[g][e] * f));
        m[g] = M;
        l[g] = lg;
    }
    static_assert(EPL % 4 == 0, "groups of four values");
    const int row = lane >> 4;
#pragma unroll
    for (int k = 0; k < GT * EPL / 4; k++) {
        const int g = (4 * k) / EPL, j = (4 * k) % EPL;  // the group's first value: head g, element slot j
        const float u = pair32(pair16(acc[g][j], acc[g][j + 1]), pair16(acc[g][j + 2], acc[g][j + 3]));
        if ((lane & 8) == 0) {
            const int jr = j + row;  // this row's value: element slot jr of head g
            lds_acc[wave][g][((jr / EPC) * 8 + sub) * EPC + jr % EPC] = u;
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < GT; g++) {
            lds_m[wave][g] = m[g];
            lds_l[wave][g] = l[g];
        }
    }
    __syncthreads();

    // merge the 4 waves; write the output or this split's partial
    const int64_t unit = ((int64_t)b * p.n_kv_heads + kvh) * p.n_hg + hg;
    const bool arrive = r.n_splits > 1 && r.n_pages <= p.merge_pages;  // a rule on the window alone
    for (int idx = tid; idx < gcount * D; idx += kThreads) {
        const int g = idx / D;
        const int e = idx - g * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, lds_m[w][g]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float mw = lds_m[w][g];
            const float f = (mw == -INFINITY) ? 0.0f : fast_exp2(mw - M);
            L = fmaf(lds_l[w][g], f, L);
            A = fmaf(lds_acc[w][g][e], f, A);
        }
        if (r.n_splits == 1) {
            p.out[((int64_t)b * p.n_heads + h_base + g) * D + e] = L > 0.0f ? A * (1.0f / L) : A;
        } else {
            const int64_t slot = unit * p.max_splits + split;
            if (arrive)
                store_agent(p.part_acc + (slot * GT + g) * D + e, A);
            else
                p.part_acc[(slot * GT + g) * D + e] = A;
        }
    }
    // (m, l) of the split's heads as one whole 128-byte line: sub-line writes cost a
    // read-modify-write in HBM (measured on the Q8_0 kernel's partials: 3-12 us per call)
    if (r.n_splits > 1 && tid < 8) {
        float M = -INFINITY, L = 0.0f;
        const int g = tid & 7;
        if (g < GT) {
#pragma unroll
            for (int w = 0; w < kWaves; w++) M = fmaxf(M, lds_m[w][g]);
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                const float mw = lds_m[w][g];
                const float f = (mw == -INFINITY) ? 0.0f : fast_exp2(mw - M);
                L = fmaf(lds_l[w][g], f, L);
            }
        }
        // lane t < 4 writes floats 4t .. 4t+3 of the line: m[0..7], l[0..7]; lanes 4..7 zeros
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int src = (4 * tid + j) & 7;  // the head whose m (tid < 2) or l (tid 2, 3) goes here
            const float m_s = __shfl(M, src), l_s = __shfl(L, src);
            v[j] = tid < 2 ? m_s : (tid < 4 ? l_s : 0.0f);
        }
        const int64_t slot = unit * p.max_splits + split;
        if (arrive) {
#pragma unroll
            for (int j = 0; j < 4; j++) store_agent(p.part_ml + slot * 32 + 4 * tid + j, v[j]);
        } else {
            *reinterpret_cast<float4 *>(p.part_ml + slot * 32 + 4 * tid) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    if (!arrive) return;
    // Short window: count this split's arrival once all of its partial has
    // reached shared memory; the unit's last workgroup merges every split.
    __shared__ int lds_last;
    if (!arrive_last(p.arrivals + unit, r.n_splits, &lds_last)) return;
    merge_splits_agent<D, GT>(p, unit * p.max_splits, r.n_splits, gcount, p.out + ((int64_t)b * p.n_heads + h_base) * D);
}

// Log-sum-exp merge of the split partials of one (sequence, kv head, head
// group, q-head g = blockIdx.x). A row of D floats is read by D/4 lanes as
// float4; the 256 threads form 256/(D/4) split groups that take every
// NSG-th split, four splits in flight at a time, and are merged through LDS.
template <int D, int GT>
__global__ __launch_bounds__(kThreads) void decode_combine_kernel(const DecodeParams p) {
    constexpr int RL = D / 4;             // lanes per row
    constexpr int NSG = kThreads / RL;    // split groups
    constexpr int BATCH = 4;
    __shared__ float4 lds_a[NSG][RL];
    __shared__ float lds_m[NSG], lds_l[NSG];

    const int b = blockIdx.z;
    const int kvh = blockIdx.y / p.n_hg;
    const int hg = blockIdx.y - kvh * p.n_hg;
    const int g = blockIdx.x;
    const int gcount = min(GT, p.group - hg * GT);
    if (g >= gcount) return;
    const SeqRange r = seq_range(p, b);
    if (r.n_splits <= 1 || r.n_pages <= p.merge_pages) return;  // (one split, or merged in the split kernel)
    const int sg = threadIdx.x / RL;
    const int e4 = threadIdx.x - sg * RL;
    const int64_t unit = ((int64_t)b * p.n_kv_heads + kvh) * p.n_hg + hg;
    const int64_t slot0 = unit * p.max_splits;

    float M = -INFINITY, L = 0.0f;
    float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = sg; s0 < r.n_splits; s0 += NSG * BATCH) {
        float mi[BATCH], li[BATCH];
        float4 ai[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; j++) {
            const int s = s0 + j * NSG;
            const int sc = s < r.n_splits ? s : s0;
            const int64_t slot = (slot0 + sc) * GT + g;
            const bool in = s < r.n_splits;
            const float lv = p.part_ml[(slot0 + sc) * 32 + 8 + g];
            const float4 av = reinterpret_cast<const float4 *>(p.part_acc + slot * D)[e4];
            // an entry past the last split reloads split s0 and adds nothing
            // (not 0 x its sums: an infinity there would make NaN)
            mi[j] = in ? p.part_ml[(slot0 + sc) * 32 + g] : -INFINITY;
            li[j] = in ? lv : 0.0f;
            ai[j] = in ? av : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        float bm = M;
#pragma unroll
        for (int j = 0; j < BATCH; j++) bm = fmaxf(bm, mi[j]);
        // (no skip when every m is -inf: a split whose scores were all NaN has
        // m = -inf and NaN sums, and they reach the output, as the reference's do)
        const float f0 = (M == -INFINITY) ? 0.0f : fast_exp2(M - bm);
        L *= f0;
        A.x *= f0;
        A.y *= f0;
        A.z *= f0;
        A.w *= f0;
#pragma unroll
        for (int j = 0; j < BATCH; j++) {
            const float f = (mi[j] == -INFINITY) ? 0.0f : fast_exp2(mi[j] - bm);
            L = fmaf(li[j], f, L);
            A.x = fmaf(ai[j].x, f, A.x);
            A.y = fmaf(ai[j].y, f, A.y);
            A.z = fmaf(ai[j].z, f, A.z);
            A.w = fmaf(ai[j].w, f, A.w);
        }
        M = bm;
    }
    lds_a[sg][e4] = A;
    if (e4 == 0) {
        lds_m[sg] = M;
        lds_l[sg] = L;
    }
    __syncthreads();
    if (sg != 0) return;
    float MM = -INFINITY;
#pragma unroll
    for (int j = 0; j < NSG; j++) MM = fmaxf(MM, lds_m[j]);
    float LL = 0.0f;
    float4 AA = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < NSG; j++) {
        const float mj = lds_m[j];
        const float f = (mj == -INFINITY) ? 0.0f : fast_exp2(mj - MM);
        const float4 aj = lds_a[j][e4];
        LL = fmaf(lds_l[j], f, LL);
        AA.x = fmaf(aj.x, f, AA.x);
        AA.y = fmaf(aj.y, f, AA.y);
        AA.z = fmaf(aj.z, f, AA.z);
        AA.w = fmaf(aj.w, f, AA.w);
    }
    const float inv = LL > 0.0f ? 1.0f / LL : 0.0f;
    const int h = kvh * p.group + hg * GT + g;
    reinterpret_cast<float4 *>(p.out + ((int64_t)b * p.n_heads + h) * D)[e4] =
        make_float4(AA.x * inv, AA.y * inv, AA.z * inv, AA.w * inv);
}

template <int D, int GT>
int launch_typed(gla_ctx *ctx, const DecodeParams &prm, dim3 grid, bool combine) {
    if (prm.softcap > 0.0f)
        hipLaunchKernelGGL((decode_split_kernel<D, GT, kStepsPerIter, true>), grid, dim3(kThreads), 0, ctx->stream,
                           prm);
    else
        hipLaunchKernelGGL((decode_split_kernel<D, GT, kStepsPerIter, false>), grid, dim3(kThreads), 0, ctx->stream,
                           prm);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "decode_split_kernel launch: %s", hipGetErrorString(e));
    if (combine) {
        hipLaunchKernelGGL((decode_combine_kernel<D, GT>), dim3(GT, grid.x, grid.z), dim3(kThreads), 0, ctx->stream,
                           prm);
        e = hipGetLastError();
        if (e != hipSuccess)
            return set_error(GLA_ERR_KERNEL, "decode_combine_kernel launch: %s", hipGetErrorString(e));
    }
    return GLA_OK;
}

// Head-group width: the registers of a lane hold GT*(D/8) q values and as
// many accumulators, so GT*D <= 512.
int pick_gt(int d, int group) {
    const int cap = 512 / d;  // 8, 4, 2
    static const int opts[] = {1, 2, 3, 4, 8};
    for (int o : opts)
        if (o <= cap && o >= group) return o;
    return cap;
}

template <int D>
int launch_d(gla_ctx *ctx, int gt, const DecodeParams &prm, dim3 grid, bool combine) {
    switch (gt) {
    case 1:
        return launch_typed<D, 1>(ctx, prm, grid, combine);
    case 2:
        return launch_typed<D, 2>(ctx, prm, grid, combine);
    case 3:
        if constexpr (D <= 128) return launch_typed<D, 3>(ctx, prm, grid, combine);
        break;
    case 4:
        if constexpr (D <= 128) return launch_typed<D, 4>(ctx, prm, grid, combine);
        break;
    case 8:
        if constexpr (D <= 64) return launch_typed<D, 8>(ctx, prm, grid, combine);
        break;
    }
    return set_error(GLA_ERR_INVALID, "no decode kernel for head_dim %d and head group %d", D, gt);
}

}  // namespace

int launch_decode(gla_ctx *ctx, const DecodeLaunch &d) {
    if (d.q8) return launch_decode_q8(ctx, d);
    const int D = d.head_dim;
    const int group = d.n_heads / d.n_kv_heads;
    const int gt = pick_gt(D, group);
    const int n_hg = (group + gt - 1) / gt;

    // pages a window can span (a start inside a page adds one)
    const int max_pages = d.max_kv_len > 0 ? (d.max_kv_len + GLA_PAGE_SIZE - 1) / GLA_PAGE_SIZE + 1 : 1;
    const int64_t units = (int64_t)d.n_seqs * d.n_kv_heads * n_hg;
    // Split sizes come from each window alone (split_pages); GLA_DECODE_PPS
    // forces one size for every window (tuning only).
    int pps_fixed = 0;
    if (const char *env = getenv("GLA_DECODE_PPS")) {
        const int v = atoi(env);
        if (v > 0) pps_fixed = v;
    }
    const int max_splits = pps_fixed > 0 ? (max_pages + pps_fixed - 1) / pps_fixed : max_splits_upto(max_pages);

    DecodeParams prm;
    prm.kv = d.kv;
    prm.pm = d.pm;
    prm.kv_start = d.kv_start;
    prm.kv_len = d.kv_len;
    prm.q = d.q;
    prm.out = d.out;
    prm.n_heads = d.n_heads;
    prm.n_kv_heads = d.n_kv_heads;
    prm.group = group;
    prm.n_hg = n_hg;
    prm.pps_fixed = pps_fixed;
    prm.max_splits = max_splits;
    prm.max_len = d.max_kv_len;
    const bool cap = d.softcap > 0.0f;
    prm.q_mul = cap ? d.scale : d.scale * kLog2e;
    prm.softcap = cap ? d.softcap : 0.0f;
    // Windows of up to merge_pages pages merge their splits in the split
    // kernel's last workgroup (no combine launch); GLA_DECODE_MERGE_PAGES sets
    // another bound (tuning only; 0: every window through the combine).
    int merge_pages = merge_max_pages(D, gt);
    if (const char *env = getenv("GLA_DECODE_MERGE_PAGES")) merge_pages = std::max(0, atoi(env));
    prm.merge_pages = merge_pages;
    prm.arrivals = nullptr;
    // Which merges the launch needs: exact from the host lengths, else from
    // the max_kv_len bound.
    bool any_short = false, any_long = false;
    if (d.kv_len_host) {
        for (int b = 0; b < d.n_seqs; b++) {
            const int n = host_seq_pages(d.kv_start_host[b], d.kv_len_host[b], d.max_kv_len, d.pm.pos_limit);
            const int pps = pps_fixed > 0 ? pps_fixed : split_pages(n);
            if (std::min((n + pps - 1) / pps, max_splits) <= 1) continue;
            if (n <= merge_pages)
                any_short = true;
            else
                any_long = true;
        }
    } else {
        any_short = max_splits > 1 && merge_pages > 0;
        any_long = max_splits > 1 && max_pages > merge_pages;
    }
    prm.part_acc = nullptr;
    prm.part_ml = nullptr;
    if (any_short) {
        int rc = decode_arrivals(ctx, d, (size_t)units, &prm.arrivals);
        if (rc != GLA_OK) return rc;
    }
    if (max_splits > 1) {
        const size_t slots = (size_t)units * max_splits;
        const size_t acc_b = slots * gt * D * sizeof(float);
        const size_t ml_b = slots * 32 * sizeof(float);
        void *scr = nullptr;
        int rc = decode_scratch(ctx, d, acc_b + ml_b, &scr);
        if (rc != GLA_OK) return rc;
        prm.part_acc = (float *)scr;
        prm.part_ml = (float *)((uint8_t *)scr + acc_b);
    }
    if (d.n_seqs > 65535) return set_error(GLA_ERR_INVALID, "decode: n_seqs %d > 65535", d.n_seqs);
    if (max_splits > 65535) return set_error(GLA_ERR_INVALID, "decode: %d splits per sequence > 65535", max_splits);
    dim3 grid(d.n_kv_heads * n_hg, max_splits, d.n_seqs);
    switch (D) {
    case 64:
        return launch_d<64>(ctx, gt, prm, grid, any_long);
    case 128:
        return launch_d<128>(ctx, gt, prm, grid, any_long);
    case 256:
        return launch_d<256>(ctx, gt, prm, grid, any_long);
    }
    return set_error(GLA_ERR_INVALID, "unsupported head_dim %d", D);
}

}  // namespace gla
