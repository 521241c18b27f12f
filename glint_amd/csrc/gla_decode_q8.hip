// gla_decode_q8.hip -- single-token decode attention over Q8_0 KV storage,
// with both products on MFMA (gfx950, v_mfma_f32_16x16x32_f16).
//
// Math: flash_attn_1d_ext (src/tensor/flash.rs:46-124) for every q-head of a
// batch, as attn_heads_cpu runs it (src/transformer/forward.rs:240-270), over
// K/V rows dequantised as KvCacheQ8::dequant_range does (src/cache/mod.rs:318-334):
// k[d] = int8 * f16 scale of its 32-element block.
//
// Why MFMA for an HBM-bound kernel: Q8_0 moves one byte per element, and
// with G q-heads per KV head every K and V element feeds G multiply-adds.
// On the VALU that is ~5 instructions per byte at G = 4, more than the vector
// ALUs retire at HBM speed. Here the VALU only turns bytes into f16 (one
// instruction per element) and applies per-token scales; the products run on
// the matrix cores.
//
// Exactness. int8 values are exact in f16. q and the probabilities are f32;
// each is split into two f16 pieces (hi = f16(x), lo = f16(x - hi)) after a
// power-of-two rescale that puts the largest magnitude below 2^14, so
// hi + lo carries ~22 significant bits and no piece is subnormal where it
// matters. The MFMA multiplies f16 pairs exactly and accumulates in f32.
//
// Work: one wave = one (sequence, KV head, group of <= 4 q-heads, chunk of
// `ch` pages); a workgroup is 4 waves on 4 consecutive chunks. A step covers
// two pages (32 positions), the K depth of one P.V MFMA.
//   S = K . Q   A = K tile (16 positions x one 32-element Q8_0 block), B = Q:
//               column j = (head (j>>1)&3, piece j&1); columns 0-7 carry the
//               even blocks and columns 8-15 the odd blocks (zero operand
//               halves), so every lane scales only its own blocks' partial
//               scores and one row rotation adds the two halves.
//   O += P' . V A = P' (row r = (page r>>3 of the step, head, piece)), B = V
//               tile (32 positions x 16 d); P'[r][t] = piece of
//               p[t] * vscale[t][block] * 2^kv. Rows of page 0 are zero on
//               page-1 positions and vice versa, so a lane builds only the
//               values of its own page and every lane's S column is exactly
//               its P' row: no data moves between lanes.
// Quants are stored sign-flipped (x + 128) in this operand order
// (gla_internal.h), so each lane's operands for a page are one contiguous
// D/4-byte span and a byte becomes an exact f16 with one permute and one
// packed subtract per two elements.
// The 4 waves of a workgroup merge their chunks (log-sum-exp) in LDS; units
// longer than a workgroup are merged by a second, small kernel.
//
// Batch invariance (the reference's batched == single guarantee,
// src/transformer/forward.rs:1946-2002): a sequence's chunks, workgroups and
// merge order depend on its own window and head_dim only, never on the rest
// of the batch. What adapts to the batch is how many q-heads a wave carries
// (hpw): a head owns its own MFMA columns (S) and rows (P'.V), its own
// maximum, sum and q scale, so its result does not depend on the heads that
// share its wave.
#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <cmath>

#include "gla_internal.h"

namespace gla {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kGT = 4;  // q-heads a wave can carry (MFMA column / row groups)
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxChunks = 64;  // preferred bound on chunks per unit
// Workgroup rows listed in the launch arguments (see Q8Params::rows): 3 KB of
// the 4 KB kernel-argument limit.
constexpr int kMaxRows = 1536;
// Floats per (unit, workgroup) partial: O, then one 128-byte line holding m and l.
template <int D>
constexpr int kPartStride = kGT * D + 32;

struct Q8Params {
    const uint8_t *base;  // KV storage; a (page, head) block is 34*D bytes
    int64_t page_stride;
    int64_t head_stride;
    PageMap pm;
    const int32_t *kv_start;
    const int32_t *kv_len;
    const float *q;
    float *out;
    float *part;  // [unit][max_wg] { O[kGT][D] (unnormalised) | m[kGT], l[kGT], zeros: 32 floats }
    int n_heads;
    int n_kv_heads;
    int group;
    int hpw;     // q-heads per wave (1..kGT)
    int n_hg;    // head groups per KV head: ceil(group / hpw)
    int ch;      // pages per chunk (even)
    int max_wg;  // workgroups per unit (partials per unit)
    int max_len;
    float q_mul;    // scale*log2(e), or scale with a soft-cap
    float softcap;  // > 0: cap * tanh(s / cap)
    // With the host lengths known: the (sequence, workgroup) of grid row y,
    // seq << 6 | wg, longest workgroups first, and no rows for workgroups
    // past a sequence's end (n_rows > 0; grid (units, n_rows, 1)). Else
    // n_rows = 0 and the grid is (units, max_wg, n_seqs).
    int n_rows;
    uint16_t rows[kMaxRows];
};

struct Range {
    int start, end;  // positions [start, end)
    int fp;          // first logical page
    int n_pages;
};

__device__ __forceinline__ Range seq_range(const Q8Params &p, int b) {
    Range r;
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
    } else {
        r.fp = 0;
        r.n_pages = 0;
    }
    return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// tanh(x) = sign(x) (1 - t) / (1 + t), t = exp(-2|x|), with the hardware
// reciprocal (1 ulp) in place of a full-precision divide.
__device__ __forceinline__ float tanh_approx(float x) {
    const float t = fast_exp2(-2.0f * kLog2e * fabsf(x));
    return copysignf((1.0f - t) * __builtin_amdgcn_rcpf(1.0f + t), x);
}

// Four stored quants (x + 128, in byte order) -> halves at..at+3 of `o`:
// 0x64XX is 1024 + XX in f16, so subtracting 1152 leaves x exactly.
__device__ __forceinline__ void q4_to_h(uint32_t u, half8 &o, int at) {
    const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const half2v a = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
    const half2v c = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
    o[at + 0] = a[0];
    o[at + 1] = a[1];
    o[at + 2] = c[0];
    o[at + 3] = c[1];
}

__device__ __forceinline__ uint32_t word(const uint4 &v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// f16 number i of a packed word array.
template <int N>
__device__ __forceinline__ float half_at(const uint32_t (&a)[N], int i) {
    const uint32_t w = a[i >> 1];
    return (float)__builtin_bit_cast(_Float16, (uint16_t)((i & 1) ? (w >> 16) : (w & 0xffff)));
}

__device__ __forceinline__ float dpp_swap1(float x) {  // lane ^ 1
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
}

__device__ __forceinline__ float dpp_ror8(float x) {  // lane ^ 8 within a row of 16
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
}

// Across the four rows of 16 lanes (lane ^ 16, lane ^ 32) with the gfx950
// row swaps: VALU only, no LDS round trip.
__device__ __forceinline__ float max_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}
__device__ __forceinline__ float sum_rows(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}
__device__ __forceinline__ float sum_halves(float x) {  // lane ^ 32
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}

typedef int int16s __attribute__((ext_vector_type(16)));

// Physical page of chunk page `lane` (0..npg-1) of sequence b, clamped into
// the pool as map_page does, read through the scalar cache. A new
// workgroup's first K/V loads wait for these ids: on the vector path the
// table read queued behind the CU's streaming loads (1.7-3.3 us for
// workgroups that start mid-kernel), on the scalar path it returns in
// 0.2-0.3 us. Each round reads two 16-entry windows of the sequence's table
// row with s_load_dwordx16, each window kept inside the row (a window that
// would pass the row's end starts earlier instead), writes them into lanes
// 0-15 of two registers and moves each chunk page's entry to its lane.
// Needs pt_stride >= 16.
__device__ __forceinline__ int chunk_ids_scalar(const PageMap &pm, int b, int pg0, int npg, int lane) {
    const int32_t *row = pm.page_table + (int64_t)b * pm.pt_stride;
    int v = 0;
#pragma unroll
    for (int g = 0; g < 64; g += 32) {
        if (g >= npg) break;
        const int w0 = min(pg0 + g, pm.pt_stride - 16);
        const int w1 = min(pg0 + g + 16, pm.pt_stride - 16);
        int16s lo, hi;
        asm volatile(
            "s_load_dwordx16 %0, %2, 0x0\n\t"
            "s_load_dwordx16 %1, %3, 0x0\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&s"(lo), "=&s"(hi)
            : "s"(row + w0), "s"(row + w1)
            : "memory");
        int tl = 0, th = 0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(tl) : "s"(lo[j]), "i"(j));
            asm volatile("v_writelane_b32 %0, %1, %2" : "+v"(th) : "s"(hi[j]), "i"(j));
        }
        const int a = __shfl(tl, min(max(pg0 + lane - w0, 0), 15));
        const int c = __shfl(th, min(max(pg0 + lane - w1, 0), 15));
        v = (lane >= g && lane < g + 16) ? a : v;
        v = (lane >= g + 16 && lane < g + 32) ? c : v;
    }
    const int last = (int)(pm.n_pages - 1);
    return v < 0 ? 0 : (v > last ? last : v);
}

// e with x = m * 2^e, m in [0.5, 1); scaling by 2^(14 - e) maps max|.| below 2^14.
__device__ __forceinline__ int pow2_exp(float x) {
    int e = 0;
    (void)frexpf(x, &e);
    return e < -100 ? -100 : (e > 100 ? 100 : e);
}

// The lane's operands of one step, in registers: the K half is read at the
// top of the step and the V half after the softmax, so only one half is live
// at a time.
template <int D>
struct RawK {
    static constexpr int NQ = D / 64;  // uint4 per lane per (page, head) K block
    static constexpr int NB = D / 32;
    uint4 k[2][NQ];
    uint32_t ks[2][NB];  // 4 positions x the lane's NB/2 blocks, per page
};
template <int D>
struct RawV {
    static constexpr int NQ = D / 64;
    static constexpr int NB = D / 32;
    uint4 v[2][NQ];
    uint32_t vs[2 * NB];  // 4 positions x NB blocks, the lane's P.V page only
};

// ---- the LDS slot: direct global -> LDS loads (gfx950 global_load_lds) ----
//
// Each wave streams its chunk through one LDS slot of two pages, in two
// halves: K = K_a | K_b | Ks_a | Ks_b and V = V_a | V_b | Vs_a | Vs_b (16*D
// bytes per quant block, byte copies of the (page, head) blocks with lane l's
// piece c at c*1024 + l*16; D bytes per scale array). At the top of a step
// the wave copies the K half into registers and refills it with the next
// step; after the softmax it does the same with the V half. Each half's next
// step is in flight for a whole step, and only one half is held in
// registers at a time.
// The loads are issued from inline assembly with explicit vmcnt waits: the
// compiler's own wait insertion would wait for every outstanding LDS load
// before any LDS read. Every vector-memory instruction of the streaming loop
// is one of these, so the counts are exact; the compiler's waits for its own
// earlier loads stay correct because extra outstanding loads only make an
// in-order wait wait longer.
constexpr int kSlotBytesPerD = 68;  // per half: 32*D quant bytes + 2*D scale bytes
constexpr int kHalfV = 34;         // the V half starts at 34*D

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// 16 bytes per lane from sbase + voff into LDS at m0 + 16*lane (m0 restored
// afterwards); sbase is wave-uniform (SGPRs), so the per-load address needs
// no 64-bit arithmetic on the VALU.
// The loads are non-temporal (nt): every byte is read once per call, and
// streaming them past the caches measured ~10% faster than default loads.
// An LDS-DMA load needs one wait state after an SALU write of M0, and the
// compiler cannot insert it into inline assembly: hence the s_nop.
__device__ __forceinline__ void dma16_s(const uint8_t *sbase, uint32_t voff, uint32_t m0) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2 nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(voff), "s"(sbase), "s"(m0)
        : "memory");
}

// 4 bytes per lane from sbase + voff into LDS at m0 + 4*lane, for the lanes
// of the 64-bit mask (mlo | mhi << 32) only; exec is restored afterwards.
__device__ __forceinline__ void dma4_s(const uint8_t *sbase, uint32_t voff, uint32_t m0, uint32_t mlo,
                                       uint32_t mhi) {
    uint64_t save_exec;
    uint32_t save_m0;
    asm volatile(
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b32 exec_lo, %4\n\t"
        "s_mov_b32 exec_hi, %5\n\t"
        "s_mov_b32 %1, m0\n\t"
        "s_mov_b32 m0, %6\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %2, %3 nt\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(save_exec), "=&s"(save_m0)
        : "v"(voff), "s"(sbase), "s"(mlo), "s"(mhi), "s"(m0)
        : "memory");
}

__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait until at most N vector-memory loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmem() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Loads per half-step: the two quant blocks in kilobyte pieces and one
// dword load per scale array.
template <int D>
constexpr int kLoadsPerHalf = 2 * (D / 64) + 2;

// Issue the loads of half V (0: K, 1: V) of step `step` (pages 2*step,
// 2*step+1 of the chunk) into the slot at LDS byte address `slot`.
template <int D, int V>
__device__ __forceinline__ void issue_half(const Q8Params &p, const uint8_t *head_base, int pid_l, int step,
                                           int npg, int lane, uint32_t slot) {
    constexpr int NQ = D / 64;
    const int pa = 2 * step;
    const int pb = (pa + 1 < npg) ? pa + 1 : pa;
    const int ida = __builtin_amdgcn_readlane(pid_l, pa);
    const int idb = __builtin_amdgcn_readlane(pid_l, pb);
    const uint8_t *ba = head_base + (int64_t)ida * p.page_stride + V * 16 * D;
    const uint8_t *bb = head_base + (int64_t)idb * p.page_stride + V * 16 * D;
    const uint32_t dst = slot + V * kHalfV * D;
    // byte copies of the quant blocks, one contiguous kilobyte per load
    const uint32_t voff = (uint32_t)lane * 16;
#pragma unroll
    for (int c = 0; c < NQ; c++) {
        dma16_s(ba + c * 1024, voff, dst + c * 1024);
        dma16_s(bb + c * 1024, voff, dst + 16 * D + c * 1024);
    }
    // scales, byte-identical: [s_a | s_b] from 32*D (K) or 33*D (V) of the
    // page-head, D bytes each = D/4 lanes of one dword. Up to d128 both fit
    // one wave-wide LDS row and go out as two lane-masked loads sharing m0.
    const uint8_t *sa = head_base + (int64_t)ida * p.page_stride + (32 + V) * D;
    const uint8_t *sb = head_base + (int64_t)idb * p.page_stride + (32 + V) * D;
    const uint32_t voff4 = (uint32_t)lane * 4;
    if constexpr (D == 256) {
        dma4_s(sa, voff4, dst + 32 * D, 0xffffffffu, 0xffffffffu);
        dma4_s(sb, voff4, dst + 32 * D + 256, 0xffffffffu, 0xffffffffu);
    } else if constexpr (D == 128) {
        dma4_s(sa, voff4, dst + 32 * D, 0xffffffffu, 0u);
        dma4_s(sb - D, voff4, dst + 32 * D, 0u, 0xffffffffu);
    } else {
        static_assert(D == 64, "head_dim 64, 128 or 256");
        dma4_s(sa, voff4, dst + 32 * D, 0x0000ffffu, 0u);
        dma4_s(sb - D, voff4, dst + 32 * D, 0xffff0000u, 0u);
    }
}

template <int N>
__device__ __forceinline__ void lds_words(const uint8_t *src, uint32_t (&dst)[N]) {
    static_assert(N % 2 == 0, "whole 8-byte reads");
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; i++) {
            const uint4 w = reinterpret_cast<const uint4 *>(src)[i];
            dst[4 * i] = w.x;
            dst[4 * i + 1] = w.y;
            dst[4 * i + 2] = w.z;
            dst[4 * i + 3] = w.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N / 2; i++) {
            const uint2 w = reinterpret_cast<const uint2 *>(src)[i];
            dst[2 * i] = w.x;
            dst[2 * i + 1] = w.y;
        }
    }
}

// Copy the lane's operands of a landed half-step from the slot.
template <int D>
__device__ __forceinline__ void read_k(const uint8_t *slot, int lane, RawK<D> &r) {
    constexpr int NQ = D / 64;
    constexpr int NB = D / 32;
    const int kg = lane >> 4;
    const int hb = (lane >> 3) & 1;  // the lane's block parity
#pragma unroll
    for (int c = 0; c < NQ; c++) {
        r.k[0][c] = *reinterpret_cast<const uint4 *>(slot + 0 * 16 * D + c * 1024 + lane * 16);
        r.k[1][c] = *reinterpret_cast<const uint4 *>(slot + 1 * 16 * D + c * 1024 + lane * 16);
    }
    // K scales: [parity][slot][NB/2] f16; the lane's 4 positions of its parity
    const uint8_t *ks = slot + 32 * D + (hb * 16 + kg * 4) * NB;
    lds_words(ks, r.ks[0]);
    lds_words(ks + D, r.ks[1]);
}
template <int D>
__device__ __forceinline__ void read_v(const uint8_t *slot, int lane, RawV<D> &r) {
    constexpr int NQ = D / 64;
    constexpr int NB = D / 32;
    const int kg = lane >> 4;
    const int hb = (lane >> 3) & 1;  // the lane's P'.V page
    const uint8_t *vh = slot + kHalfV * D;
#pragma unroll
    for (int c = 0; c < NQ; c++) {
        r.v[0][c] = *reinterpret_cast<const uint4 *>(vh + 0 * 16 * D + c * 1024 + lane * 16);
        r.v[1][c] = *reinterpret_cast<const uint4 *>(vh + 1 * 16 * D + c * 1024 + lane * 16);
    }
    // V scales: [slot][NB] f16; the lane's 4 positions of its page
    lds_words(vh + 32 * D + hb * D + kg * 4 * NB * 2, r.vs);
}

template <int D>
struct StepConst {
    half8 qb[D / 32];  // Q operand per block (zero unless the block's parity is the lane's)
    // Scores are kept in the q-scaled domain: the log2-domain score is
    // sm * s (sm = 2^(qe - 14), or 1 after a soft-cap, which is applied to
    // the true score). P' is p * 2^kvs * vscale, 2^kvs folded into the exp.
    float sm, kvs, softcap, qcap;
    bool cap;
    int pg0, npg, start, end;
    int kg, ph;
    float pf;  // this lane's piece (0: hi, 1: lo) as a float
};

template <int D>
struct StepState {
    floatx4 acc[D / 16];
    float m;     // running max (log2 domain) of the lane's head
    float lsum;  // sum of p over this lane's P' positions
};

// First half of a step (two pages, 32 positions, of one sequence and KV
// head): S = K.Q, the soft-cap, the window mask and the online softmax.
// Leaves in pr the probabilities of the lane's four P' positions and in
// vbad the positions whose V scale must be ignored (bit i).
template <int D>
__device__ __forceinline__ void step_qk(const RawK<D> &cur, int step, const StepConst<D> &c, StepState<D> &st,
                                        float (&pr)[4], int &vbad) {
    constexpr int NB = D / 32;
    constexpr int ND = D / 16;

    // S = K . Q for both pages: the lane holds positions kg*4 + i of its column
    float s0[4], s1[4];
#pragma unroll
    for (int P = 0; P < 2; P++) {
        floatx4 cp[NB / 2];
#pragma unroll
        for (int j = 0; j < NB / 2; j++) cp[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int blk = 0; blk < NB; blk++) {
            half8 a;
            q4_to_h(word(cur.k[P][blk >> 1], (blk & 1) * 2), a, 0);
            q4_to_h(word(cur.k[P][blk >> 1], (blk & 1) * 2 + 1), a, 4);
            cp[blk >> 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, c.qb[blk], cp[blk >> 1], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float x = 0.0f;
#pragma unroll
            for (int j = 0; j < NB / 2; j++) x = fmaf(half_at(cur.ks[P], i * (NB / 2) + j), cp[j][i], x);
            x += dpp_ror8(x);   // even blocks + odd blocks
            x += dpp_swap1(x);  // hi piece + lo piece
            if (P == 0)
                s0[i] = x;
            else
                s1[i] = x;
        }
    }
    if (c.cap) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s0[i] = c.softcap * tanh_approx(s0[i] * c.qcap) * kLog2e;
            s1[i] = c.softcap * tanh_approx(s1[i] * c.qcap) * kLog2e;
        }
    }

    // Window / length mask: only a chunk's first and last steps can hold
    // positions outside [start, end). Masked positions get score -inf and,
    // on the lane's own page, are flagged so that their V scale is zeroed and
    // a non-finite scale of an unused position cannot reach the output.
    vbad = 0;
    const int sp = (c.pg0 + 2 * step) * 16;             // first position of the step
    const int lim1 = min(c.end, (c.pg0 + c.npg) * 16);  // page 1 of the step may be past the chunk
    if (sp < c.start || sp + 32 > lim1) {
        const int pos0 = sp + c.kg * 4;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const bool ok0 = pos0 + i >= c.start && pos0 + i < c.end;
            const bool ok1 = pos0 + 16 + i >= c.start && pos0 + 16 + i < lim1;
            s0[i] = ok0 ? s0[i] : -INFINITY;
            s1[i] = ok1 ? s1[i] : -INFINITY;
            const bool ok = c.ph ? ok1 : ok0;
            vbad |= ok ? 0 : (1 << i);
        }
    }
    const float tmax = max_rows(fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                                      fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3]))));
    const float m_new = fmaxf(st.m, tmax);  // finite: page 0 of a step always holds a position
    const float alpha = fast_exp2((st.m - m_new) * c.sm);
    st.m = m_new;
    const float off = c.kvs - m_new * c.sm;

#pragma unroll
    for (int i = 0; i < 4; i++) pr[i] = fast_exp2(fmaf(c.ph ? s1[i] : s0[i], c.sm, off));
    st.lsum = st.lsum * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));

    if (__ballot(alpha != 1.0f)) {
        // rows kg*4 + {0,1} belong to head (2kg)&3, rows kg*4 + {2,3} to (2kg+1)&3
        const float aA = __shfl(alpha, ((2 * c.kg) & 3) * 2);
        const float aB = __shfl(alpha, ((2 * c.kg + 1) & 3) * 2);
#pragma unroll
        for (int t = 0; t < ND; t++) {
            st.acc[t][0] *= aA;
            st.acc[t][1] *= aA;
            st.acc[t][2] *= aB;
            st.acc[t][3] *= aB;
        }
    }
}

// Second half of a step: O += P' . V, one 32-element block (two d tiles) at
// a time. v = p * vscale * 2^kv; the lane's piece is f16(v - pf * f16(v)).
template <int D>
__device__ __forceinline__ void step_pv(RawV<D> &cur, const StepConst<D> &c, StepState<D> &st, const float (&pr)[4],
                                        int vbad) {
    constexpr int NB = D / 32;
    if (vbad) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int w = 0; w < NB / 2; w++)
                cur.vs[i * (NB / 2) + w] = ((vbad >> i) & 1) ? 0u : cur.vs[i * (NB / 2) + w];
    }
#pragma unroll
    for (int blk = 0; blk < NB; blk++) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = fmaf(pr[i], half_at(cur.vs, i * NB + blk), 0.0f);
        const half2v h01 = __builtin_convertvector((float2v){v[0], v[1]}, half2v);
        const half2v h23 = __builtin_convertvector((float2v){v[2], v[3]}, half2v);
        const half2v e01 = {(_Float16)fmaf(-c.pf, (float)h01[0], v[0]), (_Float16)fmaf(-c.pf, (float)h01[1], v[1])};
        const half2v e23 = {(_Float16)fmaf(-c.pf, (float)h23[0], v[2]), (_Float16)fmaf(-c.pf, (float)h23[1], v[3])};
        const uint32_t w0 = __builtin_bit_cast(uint32_t, e01);
        const uint32_t w1 = __builtin_bit_cast(uint32_t, e23);
        const uint4 pw = c.ph ? make_uint4(0u, 0u, w0, w1) : make_uint4(w0, w1, 0u, 0u);
        const half8 pa = __builtin_bit_cast(half8, pw);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int t = 2 * blk + h;
            half8 vb;
            q4_to_h(word(cur.v[0][t >> 2], t & 3), vb, 0);
            q4_to_h(word(cur.v[1][t >> 2], t & 3), vb, 4);
            st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, st.acc[t], 0, 0, 0);
        }
    }
}

// One wave's chunk: flash attention of the group's q-heads over `ch` pages;
// leaves O (unnormalised, true scale), m and l of each head at the start of
// the wave's LDS slot ([kGT][D + 2] floats).
template <int D>
__device__ __forceinline__ void wave_chunk(const Q8Params &p, const Range &r, int b, int kvh, int h_base,
                                           int gcount, int pg0, int npg, int lane, uint8_t *slot) {
    constexpr int NB = D / 32;  // Q8_0 blocks per head row
    constexpr int ND = D / 16;  // 16-wide d tiles of O
    const int kg = lane >> 4;   // lane group: MFMA k-slots kg*8 .. kg*8+7
    const int lc = lane & 15;   // S column / P' row / O column of the lane
    const int nsteps = (npg + 1) >> 1;

    // q and the chunk's page ids are loaded together (the streaming loads
    // below are a compiler barrier, so q must be requested before them)
    const int gq = (lc >> 1) & 3;  // head of this lane's column / row
    const int piece = lc & 1;
    const int ph = (lc >> 3) & 1;  // block parity of the column; page of the P' row
    const bool qvalid = gq < gcount;
    float4 qraw[NB][2];
    {
        const float *qp = p.q + ((int64_t)b * p.n_heads + h_base + (qvalid ? gq : 0)) * D;
#pragma unroll
        for (int blk = 0; blk < NB; blk++) {
            qraw[blk][0] = *reinterpret_cast<const float4 *>(qp + blk * 32 + kg * 8);
            qraw[blk][1] = *reinterpret_cast<const float4 *>(qp + blk * 32 + kg * 8 + 4);
        }
    }
    // physical page of chunk page `lane` (clamped into the pool by map_page)
    const int pid_l = p.pm.page_table && p.pm.pt_stride >= 16
                          ? chunk_ids_scalar(p.pm, b, pg0, npg, lane)
                          : (int)map_page(p.pm, b, pg0 + min(lane, npg - 1));
    const uint8_t *head_base = p.base + (int64_t)kvh * p.head_stride;

    // Start streaming the first step and request the chunk's V scales now,
    // before q is split: the compiler does not count the streaming loads, so
    // its wait for q below waits for them too, and the q, the step's K/V and
    // the scales then arrive in one round trip.
    const uint32_t slot_lds = __builtin_amdgcn_readfirstlane(lds_addr(slot));
    issue_half<D, 0>(p, head_base, pid_l, 0, npg, lane, slot_lds);
    issue_half<D, 1>(p, head_base, pid_l, 0, npg, lane, slot_lds);

    // ---- largest V scale of the chunk: P' = p * vscale * 2^kv stays below 2^14 ----
    // 16-byte units of the chunk's V scales, four loads per lane in flight per
    // batch (one batch up to 128 pages at d128)
    const int units = npg * 2 * NB;
    auto scan_loads = [&](int u0, uint4 (&w)[4]) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int uu = min(u0 + j * 64 + lane, units - 1);
            const int pid = __shfl(pid_l, uu / (2 * NB));
            w[j] = *reinterpret_cast<const uint4 *>(head_base + (int64_t)pid * p.page_stride + 33 * D +
                                                    (uu % (2 * NB)) * 16);
        }
    };
    auto scan_max = [&](const uint4 (&w)[4], float vmax) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t a[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
            for (int i = 0; i < 8; i++) vmax = fmaxf(vmax, fabsf(half_at(a, i)));
        }
        return vmax;
    };
    uint4 w0[4];
    scan_loads(0, w0);

    // ---- Q as the B operand of S = K.Q ----
    float qx[NB][8];
    float qmax = 0.0f;
#pragma unroll
    for (int blk = 0; blk < NB; blk++) {
        const float t[8] = {qraw[blk][0].x, qraw[blk][0].y, qraw[blk][0].z, qraw[blk][0].w,
                            qraw[blk][1].x, qraw[blk][1].y, qraw[blk][1].z, qraw[blk][1].w};
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const float x = t[s] * p.q_mul;
            qx[blk][s] = x;
            qmax = fmaxf(qmax, fabsf(x));
        }
    }
    qmax = max_rows(qmax);
    // An infinite q entry (a wave-uniform branch, so finite q pays nothing for
    // it): the scale comes from the finite entries and the infinity keeps its
    // own pieces exact (hi = +-inf, lo = 0), so its scores are +-inf, or +-cap
    // under the soft-cap, as the reference's are.
    const bool q_inf = __ballot(!(qmax <= 3.402823466e38f)) != 0;
    if (q_inf) {
        float fm = 0.0f;
#pragma unroll
        for (int blk = 0; blk < NB; blk++)
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const float a = fabsf(qx[blk][s]);
                fm = a <= 3.402823466e38f ? fmaxf(fm, a) : fm;
            }
        qmax = max_rows(fm);
    }
    const int qe = pow2_exp(qmax);
    const float qs = ldexpf(1.0f, 14 - qe);
    StepConst<D> c;
#pragma unroll
    for (int blk = 0; blk < NB; blk++)
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const float x = qx[blk][s] * qs;
            const _Float16 hi = (_Float16)x;
            const _Float16 lo = (_Float16)(x - (float)hi);
            const bool mine = qvalid && ((blk & 1) == ph);
            c.qb[blk][s] = mine ? (piece ? lo : hi) : (_Float16)0.0f;
        }
    if (q_inf) {
#pragma unroll
        for (int blk = 0; blk < NB; blk++)
#pragma unroll
            for (int s = 0; s < 8; s++)
                if (piece && __builtin_isinf(qx[blk][s])) c.qb[blk][s] = (_Float16)0.0f;
    }
    const float inv_qs = ldexpf(1.0f, qe - 14);

    float inv_vsc;
    {
        float vmax = scan_max(w0, 0.0f);
        for (int u0 = 256; u0 < units; u0 += 256) {
            uint4 w[4];
            scan_loads(u0, w);
            vmax = scan_max(w, vmax);
        }
        vmax = wave_max(vmax);
        const int ve = pow2_exp(vmax);
        c.kvs = (float)(14 - ve);
        inv_vsc = ldexpf(1.0f, ve - 14);
    }

    c.cap = p.softcap > 0.0f;
    c.softcap = p.softcap;
    c.qcap = c.cap ? inv_qs / p.softcap : 0.0f;
    c.sm = c.cap ? 1.0f : inv_qs;
    c.pg0 = pg0;
    c.npg = npg;
    c.start = r.start;
    c.end = r.end;
    c.kg = kg;
    c.ph = ph;
    c.pf = (float)piece;

    StepState<D> st;
#pragma unroll
    for (int t = 0; t < ND; t++) st.acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    st.m = -INFINITY;
    st.lsum = 0.0f;

    constexpr int NL = kLoadsPerHalf<D>;
    for (int step = 0; step < nsteps; step++) {
        const bool next = step + 1 < nsteps;
        wait_vmem<NL>();  // the K half of `step` has landed (its V half may not have)
        RawK<D> kr;
        read_k<D>(slot, lane, kr);
        if (next) {
            wait_lds();  // the K half is copied: refill it with the next step
            issue_half<D, 0>(p, head_base, pid_l, step + 1, npg, lane, slot_lds);
        }
        float pr[4];
        int vbad;
        step_qk<D>(kr, step, c, st, pr, vbad);
        // the V half of `step` has landed; only the next K half may be in flight
        if (next)
            wait_vmem<NL>();
        else
            wait_vmem<0>();
        RawV<D> vr;
        read_v<D>(slot, lane, vr);
        if (next) {
            wait_lds();
            issue_half<D, 1>(p, head_base, pid_l, step + 1, npg, lane, slot_lds);
        }
        step_pv<D>(vr, c, st, pr, vbad);
    }
    wait_vmem_all();

    // ---- per-head totals ----
    // l of head gq: add the two pages (lane ^ 8) and the four lane groups
    const float L = sum_rows(st.lsum + dpp_ror8(st.lsum)) * inv_vsc;
    // O of heads gA = 2*(kg&1), gB = gA + 1 in lanes kg = 0, 1: add pieces
    // (row pairs) and the page-1 rows held by lane group kg + 2
    const int gA = (2 * kg) & 3;
    const int gB = gA + 1;
    float oA[ND], oB[ND];
#pragma unroll
    for (int t = 0; t < ND; t++) {
        oA[t] = sum_halves(st.acc[t][0] + st.acc[t][1]);
        oB[t] = sum_halves(st.acc[t][2] + st.acc[t][3]);
    }
    const float LA = __shfl(L, gA * 2), LB = __shfl(L, gB * 2);
    const float m_true = st.m * c.sm;  // log2 domain
    const float mA = __shfl(m_true, gA * 2), mB = __shfl(m_true, gB * 2);

    // the slot is idle now (every load has landed): it holds this wave's
    // result for the workgroup merge
    float *res = reinterpret_cast<float *>(slot);
    if (lane < 32) {
#pragma unroll
        for (int t = 0; t < ND; t++) {
            res[gA * (D + 2) + t * 16 + lc] = oA[t] * inv_vsc;
            res[gB * (D + 2) + t * 16 + lc] = oB[t] * inv_vsc;
        }
        if (lc == 0) {
            res[gA * (D + 2) + D] = mA;
            res[gA * (D + 2) + D + 1] = LA;
            res[gB * (D + 2) + D] = mB;
            res[gB * (D + 2) + D + 1] = LB;
        }
    }
}

// One workgroup item: (sequence b, its workgroup wg, KV head x head group hx).
// The 4 waves take 4 consecutive chunks of the unit and merge them in LDS; a
// unit longer than one workgroup writes one partial per workgroup.
template <int D>
__device__ __forceinline__ void q8_item(const Q8Params &p, uint8_t (*slots)[kSlotBytesPerD * D], int b, int wg,
                                        int hx) {
    constexpr int kThreads = kWaves * 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = hx / p.n_hg;
    const int hg = hx - kvh * p.n_hg;
    const int g0 = hg * p.hpw;
    const int gcount = min(p.hpw, p.group - g0);
    const int h_base = kvh * p.group + g0;
    float *out = p.out + ((int64_t)b * p.n_heads + h_base) * D;

    const Range r = seq_range(p, b);
    if (r.n_pages == 0) {  // empty window: zero output (the reference's pre-zeroed buffer)
        if (wg == 0)
            for (int idx = tid; idx < gcount * D; idx += kThreads) out[idx] = 0.0f;
        return;
    }
    // A workgroup covers kWaves * ch pages of the unit (the last one what is
    // left) and splits them evenly over its waves, so the waves of the
    // sequence's last, short workgroup finish together instead of one wave
    // working while the others wait at the merge.
    const int span = kWaves * p.ch;
    // (at most max_wg: partial slots are sized from the host lengths, and a
    // caller whose host copies disagree with the device arrays gets a wrong
    // result, never an access outside the slots)
    const int n_wg = min((r.n_pages + span - 1) / span, p.max_wg);
    if (wg >= n_wg) return;
    const int wg_pages = min(span, r.n_pages - wg * span);
    const int per_wave = ((wg_pages + 2 * kWaves - 1) / (2 * kWaves)) * 2;  // even: a step is two pages
    const int my0 = wave * per_wave;
    if (my0 < wg_pages) {
        wave_chunk<D>(p, r, b, kvh, h_base, gcount, r.fp + wg * span + my0, min(per_wave, wg_pages - my0), lane,
                      slots[wave]);
    } else if (lane < kGT) {
        float *res = reinterpret_cast<float *>(slots[wave]);
        res[lane * (D + 2) + D] = -INFINITY;
        res[lane * (D + 2) + D + 1] = 0.0f;
    }
    __syncthreads();
    auto res = [&](int w, int g, int i) -> float {
        return reinterpret_cast<const float *>(slots[w])[g * (D + 2) + i];
    };

    // merge the workgroup's waves; thread -> (head g, elements d .. d+3)
    const int64_t unit = ((int64_t)b * p.n_kv_heads + kvh) * p.n_hg + hg;
    float *mine = p.part + (unit * p.max_wg + wg) * kPartStride<D>;
    float Mg = -INFINITY, Lg = 0.0f;  // (M, L) of head tid, for the (m, l) line
    if (tid < kGT) {
#pragma unroll
        for (int w = 0; w < kWaves; w++) Mg = fmaxf(Mg, res(w, tid, D));
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float mw = res(w, tid, D), lw = res(w, tid, D + 1);
            if (mw != -INFINITY || lw != 0.0f) Lg = fmaf(lw, mw == -INFINITY ? 0.0f : fast_exp2(mw - Mg), Lg);
        }
    }
    for (int i4 = tid; i4 < kGT * D / 4; i4 += kThreads) {
        const int g = (4 * i4) / D;
        const int d = 4 * i4 - g * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, res(w, g, D));
        float L = 0.0f;
        float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        // A wave with no pages leaves m = -inf, l = 0 and its sums unwritten:
        // it is skipped. A wave whose scores were all NaN has m = -inf and
        // NaN l and sums: it enters with weight 0, so the NaN reaches the
        // output, as the reference's does.
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float mw = res(w, g, D);
            if (mw != -INFINITY || res(w, g, D + 1) != 0.0f) {
                const float f = mw == -INFINITY ? 0.0f : fast_exp2(mw - M);
                L = fmaf(res(w, g, D + 1), f, L);
                A.x = fmaf(res(w, g, d + 0), f, A.x);
                A.y = fmaf(res(w, g, d + 1), f, A.y);
                A.z = fmaf(res(w, g, d + 2), f, A.z);
                A.w = fmaf(res(w, g, d + 3), f, A.w);
            }
        }
        if (n_wg == 1) {
            const float inv = L > 0.0f ? 1.0f / L : 0.0f;
            if (g < gcount)
                *reinterpret_cast<float4 *>(out + g * D + d) = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
        } else {
            *reinterpret_cast<float4 *>(mine + g * D + d) = A;
        }
    }
    // The (m, l) of the partial fill one whole 128-byte line: m[kGT], l[kGT], zeros. (Partial
    // lines, and the partials' rows at a 520-byte stride, measured 3-12 us slower per cfg3 call:
    // sub-line writes cost a read-modify-write in HBM.)
    if (n_wg > 1 && tid < 8) {
        const float Ms = __shfl(Mg, tid & 3), Ls = __shfl(Lg, tid & 3);
        const float v = tid < kGT ? Ms : Ls;
        const float a0 = __shfl(v, 0), a1 = __shfl(v, 1), a2 = __shfl(v, 2), a3 = __shfl(v, 3);
        const float b0 = __shfl(v, 4), b1 = __shfl(v, 5), b2 = __shfl(v, 6), b3 = __shfl(v, 7);
        float4 line = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (tid == 0) line = make_float4(a0, a1, a2, a3);
        if (tid == 1) line = make_float4(b0, b1, b2, b3);
        *reinterpret_cast<float4 *>(mine + kGT * D + 4 * tid) = line;
    }
    // Units with more than one workgroup are merged by decode_q8_combine_kernel.
    // (Merging here in the last workgroup to finish needs a device-scope
    // release per workgroup; on gfx950 that is an L2 writeback each time and
    // measured ~6x slower than the extra launch.)
}


// Grid (KV head x head group, workgroup of the sequence, sequence), or with
// the host lengths (KV head x head group, row of the longest-first list).
// The head index runs fastest, so the workgroups reading the 8 head spans of
// the same pages are dispatched together and the DRAM rows those pages open
// are read out while open (measured ~25% over chunk-fastest order).
template <int D>
__global__ __launch_bounds__(kWaves * 64) void decode_q8_mfma_kernel(const Q8Params p) {
    // per wave: the streaming slot, later the wave's [kGT][D + 2] result
    __shared__ __attribute__((aligned(16))) uint8_t slots[kWaves][kSlotBytesPerD * D];
    static_assert(kGT * (D + 2) * 4 <= kSlotBytesPerD * D, "the merge result fits in the slot");
    int b, wg;
    if (p.n_rows > 0) {
        const int e = p.rows[blockIdx.y];
        b = e >> 6;
        wg = e & 63;
    } else {
        b = blockIdx.z;
        wg = blockIdx.y;
    }
    q8_item<D>(p, slots, b, wg, blockIdx.x);
}

// Merge of the workgroup partials of every unit with more than one
// workgroup; grid (KV head x head group, sequence), kGT*D/4 threads, each
// merging four consecutive elements of one head (16-byte loads of the
// partials; the per-element arithmetic is that of a scalar merge: eight
// partials at a time, all loads of a batch in flight together, (M, L, A)
// absorbing the batch with one rescale).
template <int D>
__global__ __launch_bounds__(kGT * D / 4) void decode_q8_combine_kernel(const Q8Params p) {
    const int b = blockIdx.y;
    const int kvh = blockIdx.x / p.n_hg;
    const int hg = blockIdx.x - kvh * p.n_hg;
    const int g0 = hg * p.hpw;
    const int gcount = min(p.hpw, p.group - g0);
    const int h_base = kvh * p.group + g0;
    const Range r = seq_range(p, b);
    const int span = kWaves * p.ch;  // pages per workgroup
    const int n_wg = min((r.n_pages + span - 1) / span, p.max_wg);
    if (n_wg <= 1) return;
    const int g = (4 * (int)threadIdx.x) / D;
    const int d = 4 * (int)threadIdx.x - g * D;
    if (g >= gcount) return;
    const int64_t unit = ((int64_t)b * p.n_kv_heads + kvh) * p.n_hg + hg;
    constexpr int64_t pstride = kPartStride<D>;
    const float *hp = p.part + unit * p.max_wg * pstride;
    float M = -INFINITY, L = 0.0f;
    float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int i0 = 0; i0 < n_wg; i0 += 8) {
        float mi[8], li[8];
        float4 ai[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = min(i0 + j, n_wg - 1);
            const bool in = i0 + j < n_wg;
            const float lv = hp[i * pstride + kGT * D + kGT + g];
            const float4 av = *reinterpret_cast<const float4 *>(hp + i * pstride + g * D + d);
            // an entry past the last partial reloads the last one and adds
            // nothing (not 0 x its sums: an infinity there would make NaN)
            mi[j] = in ? hp[i * pstride + kGT * D + g] : -INFINITY;
            li[j] = in ? lv : 0.0f;
            ai[j] = in ? av : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        float bm = M;
#pragma unroll
        for (int j = 0; j < 8; j++) bm = fmaxf(bm, mi[j]);
        // (no skip when every m is -inf: a partial whose scores were all NaN
        // has m = -inf and NaN sums, and they reach the output, as the reference's do)
        const float f0 = (M == -INFINITY) ? 0.0f : fast_exp2(M - bm);
        L *= f0;
        A.x *= f0;
        A.y *= f0;
        A.z *= f0;
        A.w *= f0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float f = (mi[j] == -INFINITY) ? 0.0f : fast_exp2(mi[j] - bm);
            L = fmaf(li[j], f, L);
            A.x = fmaf(ai[j].x, f, A.x);
            A.y = fmaf(ai[j].y, f, A.y);
            A.z = fmaf(ai[j].z, f, A.z);
            A.w = fmaf(ai[j].w, f, A.w);
        }
        M = bm;
    }
    // (L not > 0: no weight reached the head, or a NaN did; A is then 0 or NaN
    // and is written as it is, as flash.rs:118-123 leaves the sums unnormalised)
    const float inv = L > 0.0f ? 1.0f / L : 1.0f;
    *reinterpret_cast<float4 *>(p.out + ((int64_t)b * p.n_heads + h_base + g) * D + d) =
        make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
}

template <int D>
int launch_d(gla_ctx *ctx, const Q8Params &prm, dim3 grid, int n_seqs) {
    hipLaunchKernelGGL((decode_q8_mfma_kernel<D>), grid, dim3(kWaves * 64), 0, ctx->stream, prm);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "decode_q8_mfma_kernel launch: %s", hipGetErrorString(e));
    if (prm.max_wg > 1) {
        hipLaunchKernelGGL((decode_q8_combine_kernel<D>), dim3(prm.n_kv_heads * prm.n_hg, n_seqs), dim3(kGT * D / 4),
                           0, ctx->stream, prm);
        e = hipGetLastError();
        if (e != hipSuccess)
            return set_error(GLA_ERR_KERNEL, "decode_q8_combine_kernel launch: %s", hipGetErrorString(e));
    }
    return GLA_OK;
}

// Workgroups of decode_q8_mfma_kernel<D> one CU holds at once (0 on error).
template <int D>
int resident_wgs() {
    static int cached = -1;
    if (cached < 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_q8_mfma_kernel<D>, kWaves * 64, 0) != hipSuccess)
            n = 0;
        cached = n;
    }
    return cached;
}

// Pages per chunk: 28 (14 steps) for head_dim up to 128, 40 for 256, for
// every window (a chunk holds at most 64 pages, one page id per lane).
// Measured on the Llama-3-8B and Gemma-2-9B batch decodes with the workgroups
// dispatched longest first: shorter chunks repeat the q / page-id / V-scale
// set-up more often, longer ones leave the grid's last workgroups running
// alone. Fixed rather than fitted to the batch, so that a sequence's result
// is the same in any batch.
int chunk_pages(int D) { return D == 256 ? 40 : 28; }

// q-heads per wave: kGT (or the group, if smaller), lowered only while the
// workgroups that result still fit the device's resident slots in one round.
// Fewer heads per wave multiply the workgroups of a small batch (each (page,
// KV head) span is then read by group / hpw waves, dispatched together, the
// later reads served by L2), at the price of repeating the per-wave work; a
// batch that already fills most of the slots loses by it (Gemma-2's 4096
// window at B=32, 410 workgroups on 512 slots: 165 against ~110 us).
int choose_hpw(int group, int64_t wg_per_hg, int n_kv_heads, int64_t slots) {
    int hpw = std::min(kGT, group);
    int n_hg = (group + hpw - 1) / hpw;
    while (hpw > 1) {
        // the next head-group count that lowers the heads per wave (balanced
        // groups: 4 heads go 4 -> 2 + 2 -> 1 + 1 + 1 + 1)
        int h = hpw, m = n_hg;
        while (h == hpw) {
            m++;
            h = (group + m - 1) / m;
        }
        m = (group + h - 1) / h;
        if (wg_per_hg * n_kv_heads * m > slots) break;
        hpw = h;
        n_hg = m;
    }
    return hpw;
}

}  // namespace

int launch_decode_q8(gla_ctx *ctx, const DecodeLaunch &d) {
    const int D = d.head_dim;
    const int group = d.n_heads / d.n_kv_heads;
    // pages a window can span (a start inside a page adds one)
    const int64_t max_pages = d.max_kv_len > 0 ? (d.max_kv_len + GLA_PAGE_SIZE - 1) / GLA_PAGE_SIZE + 1 : 1;
    const bool host = d.kv_len_host != nullptr;
    auto pages_of = [&](int b) -> int {
        return host ? host_seq_pages(d.kv_start_host[b], d.kv_len_host[b], d.max_kv_len, d.pm.pos_limit)
                    : (int)max_pages;
    };
    // Chunk size (pages per wave; even, at most 64). GLA_Q8_CHUNK_PAGES
    // forces another size (tuning and tests).
    int ch = chunk_pages(D);
    if (const char *env = getenv("GLA_Q8_CHUNK_PAGES")) {
        const int v = atoi(env);
        if (v > 0) ch = std::min(64, (v + 1) & ~1);
    }
    const int span = kWaves * ch;  // pages per workgroup
    // workgroups per unit: exact with host lengths, else the max_kv_len bound
    int64_t max_wg = 1, wg_total = 0;
    for (int b = 0; b < d.n_seqs; b++) {
        const int64_t nw = ((int64_t)pages_of(b) + span - 1) / span;
        max_wg = std::max(max_wg, nw);
        wg_total += std::max<int64_t>(nw, 1);
    }
    const int per_cu = D == 64 ? resident_wgs<64>() : (D == 128 ? resident_wgs<128>() : resident_wgs<256>());
    const int64_t slots = (int64_t)std::max(ctx->n_cu, 1) * std::max(per_cu, 1);
    int hpw = choose_hpw(group, wg_total, d.n_kv_heads, slots);
    if (const char *env = getenv("GLA_Q8_HEADS_PER_WAVE")) {
        const int v = atoi(env);
        if (v > 0) hpw = std::min(std::min(v, kGT), group);
    }
    const int n_hg = (group + hpw - 1) / hpw;
    const int64_t units = (int64_t)d.n_seqs * d.n_kv_heads * n_hg;

    Q8Params prm;
    prm.base = d.kv.k;
    prm.page_stride = d.kv.page_stride;
    prm.head_stride = d.kv.head_stride;
    prm.pm = d.pm;
    prm.kv_start = d.kv_start;
    prm.kv_len = d.kv_len;
    prm.q = d.q;
    prm.out = d.out;
    prm.n_heads = d.n_heads;
    prm.n_kv_heads = d.n_kv_heads;
    prm.group = group;
    prm.hpw = hpw;
    prm.n_hg = n_hg;
    prm.ch = ch;
    prm.max_wg = (int)std::min<int64_t>(max_wg, 1 << 30);
    prm.max_len = d.max_kv_len;
    const bool cap = d.softcap > 0.0f;
    prm.q_mul = cap ? d.scale : d.scale * kLog2e;
    prm.softcap = cap ? d.softcap : 0.0f;
    prm.part = nullptr;
    if (d.n_seqs > 65535) return set_error(GLA_ERR_INVALID, "decode: n_seqs %d > 65535", d.n_seqs);
    if (max_wg > 65535)
        return set_error(GLA_ERR_INVALID, "decode: %lld workgroups per sequence > 65535", (long long)max_wg);
    if (max_wg > 1) {
        const size_t bytes = (size_t)units * max_wg * (kGT * D + 32) * sizeof(float);
        void *scr = nullptr;
        int rc = decode_scratch(ctx, d, bytes, &scr);
        if (rc != GLA_OK) return rc;
        prm.part = (float *)scr;
    }
    dim3 grid(d.n_kv_heads * n_hg, (unsigned)max_wg, d.n_seqs);
    // With the host lengths, list the workgroups that have pages (plus one per
    // empty window, which zeroes its output), longest first: the dispatcher
    // then starts the full workgroups before the short last ones of each
    // sequence, which fill in at the end. A counting sort over the page
    // counts (0 .. span) keeps the order stable and allocates nothing.
    prm.n_rows = 0;
    if (host && max_wg <= 64 && d.n_seqs <= 1024 && wg_total <= kMaxRows) {
        int count[4 * 64 + 2] = {0};  // rows per page count, span <= 256
        auto wg_pages = [&](int n, int j) { return n == 0 ? 0 : std::min(span, n - j * span); };
        for (int b = 0; b < d.n_seqs; b++) {
            const int n = pages_of(b);
            for (int j = 0; j == 0 || j * span < n; j++) count[wg_pages(n, j)]++;
        }
        int at[4 * 64 + 2];  // first row of each page count, longest first
        int next = 0;
        for (int c = span; c >= 0; c--) {
            at[c] = next;
            next += count[c];
        }
        for (int b = 0; b < d.n_seqs; b++) {
            const int n = pages_of(b);
            for (int j = 0; j == 0 || j * span < n; j++) prm.rows[at[wg_pages(n, j)]++] = (uint16_t)(b << 6 | j);
        }
        prm.n_rows = next;
        grid = dim3(d.n_kv_heads * n_hg, (unsigned)next, 1);
    }
    switch (D) {
    case 64:
        return launch_d<64>(ctx, prm, grid, d.n_seqs);
    case 128:
        return launch_d<128>(ctx, prm, grid, d.n_seqs);
    case 256:
        return launch_d<256>(ctx, prm, grid, d.n_seqs);
    }
    return set_error(GLA_ERR_INVALID, "unsupported head_dim %d", D);
}

}  // namespace gla
