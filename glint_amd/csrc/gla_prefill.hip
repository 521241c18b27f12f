// gla_prefill.hip -- batched causal prefill attention on MFMA (gfx950).
//
// Math: for every query row, flash_attn_1d_ext over [window_start, pos]
// (src/transformer/forward.rs:927-958, src/tensor/flash.rs:46-124).
//
// Tiling. A workgroup (4 waves) owns a block of query rows of one sequence
// and HPW q-heads that share one KV head; every wave owns 16*NT queries of one
// head. K/V tiles of KT=32 positions are staged in LDS once per workgroup and
// read by all waves (GQA reuse). Per wave and tile:
//   S^T[key][query] = K . Q^T      v_mfma_f32_16x16x4_f32, Q^T held in VGPRs
//   online softmax per query column (log2 domain)
//   O^T[d][query]  += V^T . P^T    P^T is the S^T accumulator itself: the
//                                  k-step i of a 16-key tile takes keys
//                                  {4j + i}, j = lane / 16, which is exactly
//                                  what accumulator register i holds.
// Permuting the reduction index this way costs nothing and avoids any
// register shuffle between the two products.
#include <math.h>

#include "gla_internal.h"

namespace gla {

namespace {

constexpr int KT = 32;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct PrefillParams {
    KvLayout kv;
    PageMap pm;
    const int32_t *q_start;
    const int32_t *pos_offset;
    const float *q;
    float *out;
    int n_heads;
    int n_kv_heads;
    int group;
    int hpw;           // q-heads per workgroup
    int n_qblocks;     // grid.x
    int max_q_len;     // per-sequence query counts are clamped to it
    float q_mul;       // scale*log2(e), or scale with a soft-cap
    float softcap;     // > 0: cap * tanh(s / cap)
    int sliding_window;
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max of two floats as IEEE-754 maximum (a NaN operand gives NaN): gfx950
// has v_maximum3_f32, which needs no NaN-quieting max per operand the way
// fmaxf does after a row swap or a select. Not inline asm: the compiler
// inserts the wait states an MFMA result needs before a VALU read only for
// instructions it emits itself, and these maxima read MFMA results directly.
__device__ __forceinline__ float max2f(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max / sum over the four 16-lane rows (lane ^ 16, lane ^ 32) with the gfx950
// row swaps: VALU only, no LDS round trip.
__device__ __forceinline__ float max_rows4(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = max2f(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max2f(__uint_as_float(c[0]), __uint_as_float(c[1]));
}
__device__ __forceinline__ float sum_rows4(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

__device__ __forceinline__ float tanh_approx(float x) {
    float t = fast_exp2(-2.0f * kLog2e * fabsf(x));
    float r = (1.0f - t) / (1.0f + t);
    return copysignf(r, x);
}

// Soft-cap and causal/window mask of one query column of a 32-key score tile
// (sacc[mt][i]: key k0 + 16*mt + 4*lgrp + i), in place, log2 domain. The
// soft-cap is a template argument and the mask one wave-uniform branch per
// tile with selects inside: written per score, both conditions became a
// branch around every score.
template <bool CAP>
__device__ __forceinline__ void cap_and_mask(floatx4 (&s)[2], float softcap, bool interior, int kbase, int qpos,
                                             int qlo, int klo, int khi) {
    if constexpr (CAP) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) s[mt][i] = softcap * tanh_approx(s[mt][i] / softcap) * kLog2e;
    }
    if (!interior) {
        const int lo = max(qlo, klo), hi = min(qpos, khi);
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kp = kbase + mt * 16 + i;
                s[mt][i] = (kp >= lo && kp <= hi) ? s[mt][i] : -INFINITY;
            }
    }
}

__device__ __forceinline__ int window_lo(int pos, int w) {
    if (w <= 0) return 0;
    int s = pos - w + 1;
    return s > 0 ? s : 0;
}

// One tile's K/V as f32 in registers: thread u of the workgroup holds 16
// consecutive elements (unit u / (D/16) is the key, unit % (D/16) the
// 16-element column block) of K and of V; keys outside [klo, khi] are zero.
template <int D, int NTHR>
struct TileRegs {
    static constexpr int UNITS = KT * D / 16;
    static constexpr int PER_THREAD = (UNITS + NTHR - 1) / NTHR;
    float4 k[PER_THREAD][4];
    float4 v[PER_THREAD][4];
};

template <int D, int NTHR, bool Q8>
__device__ __forceinline__ void fetch_tile(const PrefillParams &p, int b, int kvh, int k0, int klo, int khi,
                                           TileRegs<D, NTHR> &t) {
    const int64_t head_off = (int64_t)kvh * p.kv.head_stride;
#pragma unroll
    for (int j = 0; j < TileRegs<D, NTHR>::PER_THREAD; j++) {
        const int u = threadIdx.x + j * NTHR;
        const int key = u / (D / 16);
        const int c16 = u - key * (D / 16);
        const int kp = k0 + key;
        float kf[16], vf[16];
        if (u < TileRegs<D, NTHR>::UNITS && kp >= klo && kp <= khi) {
            const int64_t pid = map_page(p.pm, b, kp >> 4);
            const int slot = kp & 15;
            if constexpr (Q8) {
                // quants in the decode kernel's MFMA operand order (gla_internal.h)
                const int64_t hb = pid * p.kv.page_stride + head_off;
                const uint2 ka = *reinterpret_cast<const uint2 *>(p.kv.k + hb + q8k_off(slot, c16 * 16, D));
                const uint2 kb = *reinterpret_cast<const uint2 *>(p.kv.k + hb + q8k_off(slot, c16 * 16 + 8, D));
                const uint4 kq = make_uint4(ka.x, ka.y, kb.x, kb.y);
                uint32_t vw4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int e = 0; e < 16; e++)
                    vw4[e >> 2] |= (uint32_t)p.kv.v[hb + q8v_off(slot, c16 * 16 + e, D)] << ((e & 3) * 8);
                const int blk = (c16 * 16) >> 5;
                const uint16_t *ksp = reinterpret_cast<const uint16_t *>(p.kv.ks + hb) + q8ks_off(slot, blk, D);
                const uint16_t *vsp = reinterpret_cast<const uint16_t *>(p.kv.vs + hb) + slot * (D / 32) + blk;
                const float ksc = __half2float(__ushort_as_half(*ksp));
                const float vsc = __half2float(__ushort_as_half(*vsp));
                const uint32_t kw[4] = {kq.x, kq.y, kq.z, kq.w};
#pragma unroll
                for (int e = 0; e < 16; e++) {  // stored quants are x + 128
                    kf[e] = (float)((int)((kw[e >> 2] >> ((e & 3) * 8)) & 0xff) - 128) * ksc;
                    vf[e] = (float)((int)((vw4[e >> 2] >> ((e & 3) * 8)) & 0xff) - 128) * vsc;
                }
            } else {
                const int64_t base = pid * p.kv.page_stride + head_off + (int64_t)slot * p.kv.row_stride;
                // chunk q of the lane: floats 4*c16 + q*D/4 of the row, so
                // each load and each LDS store instruction covers whole
                // 128-byte runs of a row (16 consecutive floats per lane
                // made the LDS stores conflict)
                const float4 *kp4 = reinterpret_cast<const float4 *>(p.kv.k + base) + c16;
                const float4 *vp4 = reinterpret_cast<const float4 *>(p.kv.v + base) + c16;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    t.k[j][q] = kp4[q * (D / 16)];
                    t.v[j][q] = vp4[q * (D / 16)];
                }
                continue;
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                t.k[j][q] = make_float4(kf[4 * q], kf[4 * q + 1], kf[4 * q + 2], kf[4 * q + 3]);
                t.v[j][q] = make_float4(vf[4 * q], vf[4 * q + 1], vf[4 * q + 2], vf[4 * q + 3]);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                t.k[j][q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                t.v[j][q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
    }
}

// K and V rows in LDS: D floats + 4 of padding, so the 16 rows a 16-lane
// group reads with 16-byte loads start in distinct bank groups.
template <int D>
constexpr int kRow = D + 4;

template <int D, int NTHR, bool Q8>
__device__ __forceinline__ void store_tile(const TileRegs<D, NTHR> &t, float *Ks, float *Vs) {
#pragma unroll
    for (int j = 0; j < TileRegs<D, NTHR>::PER_THREAD; j++) {
        const int u = threadIdx.x + j * NTHR;
        if (u >= TileRegs<D, NTHR>::UNITS) break;
        const int key = u / (D / 16);
        const int c16 = u - key * (D / 16);
        // chunk q: floats 16*c16 + 4*q of the row (Q8) or 4*c16 + q*D/4 (f32)
        float4 *kd = reinterpret_cast<float4 *>(Ks + key * kRow<D> + (Q8 ? c16 * 16 : c16 * 4));
        float4 *vd = reinterpret_cast<float4 *>(Vs + key * kRow<D> + (Q8 ? c16 * 16 : c16 * 4));
#pragma unroll
        for (int q = 0; q < 4; q++) {
            kd[Q8 ? q : q * (D / 16)] = t.k[j][q];
            vd[Q8 ? q : q * (D / 16)] = t.v[j][q];
        }
    }
}

// Workgroup: NW waves; a wave owns 16*NT queries of one q-head, the HPW
// heads of the workgroup share one KV head (NW / HPW waves per head). K/V tiles of KT keys are
// double-buffered in LDS: the next tile is fetched into registers while the
// current one is multiplied, then stored to the other buffer, with one
// barrier per tile.
// Reduction order. Lane group g (lanes 16g..16g+15) covers the head
// dimensions [g*D/4, (g+1)*D/4): k-step s of S^T = K.Q^T multiplies d =
// g*D/4 + s, so a lane reads its K operands four at a time from one row.
// O^T row R of d-tile t is d = R*DT + t, so the V^T operands a lane needs
// for one key are DT consecutive floats, and a lane's outputs for a query
// are the 4*DT consecutive floats [4g*DT, 4(g+1)*DT).
template <int D, int NT, int NW, bool Q8, bool CAP>
__global__ __launch_bounds__(NW * 64) void prefill_f32_kernel(const PrefillParams p) {
    constexpr int NTHR = NW * 64;
    constexpr int QW = 16 * NT;  // queries per wave
    constexpr int KS = D / 4;    // k-steps of S = K Q^T
    constexpr int DT = D / 16;   // d tiles of O
    __shared__ __attribute__((aligned(16))) float Ks[2][KT * kRow<D>];
    __shared__ __attribute__((aligned(16))) float Vs[2][KT * kRow<D>];

    // grid (sequence x KV head x head group, query block): every unit's
    // longest (last) query block is dispatched before any shorter one, so the
    // grid ends on short workgroups
    const int n_hgrp = p.group / p.hpw;
    const int unit = blockIdx.x;
    const int b = unit / (p.n_kv_heads * n_hgrp);
    const int kvh = (unit - b * p.n_kv_heads * n_hgrp) / n_hgrp;
    const int hgrp = unit - (b * p.n_kv_heads + kvh) * n_hgrp;
    const int qblk = p.n_qblocks - 1 - (int)blockIdx.y;
    const int waves_per_head = NW / p.hpw;
    const int qwg = QW * waves_per_head;

    const int row0 = p.q_start[b];
    const int q_len = min(max(p.q_start[b + 1] - row0, 0), p.max_q_len);
    const int pos0 = p.pos_offset[b];
    const int qb0 = qblk * qwg;  // first local query of the workgroup
    if (qb0 >= q_len) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lrow = lane & 15;
    const int lgrp = lane >> 4;
    const int head = kvh * p.group + hgrp * p.hpw + (wave % p.hpw);
    const int wq0 = qb0 + (wave / p.hpw) * QW;  // first local query of this wave

    // key range of the workgroup
    const int q_last = min(q_len, qb0 + qwg) - 1;
    const int khi = min(pos0 + q_last, p.pm.pos_limit - 1);
    const int klo = window_lo(pos0 + qb0, p.sliding_window);

    // Q^T fragments: qf[nt][s] = Q[query nt*16 + lrow][d = lgrp*KS + s]
    float qf[NT][KS];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int lq = wq0 + nt * 16 + lrow;
        const bool ok = lq < q_len;
        const float4 *qp = reinterpret_cast<const float4 *>(
            p.q + ((int64_t)(row0 + (ok ? lq : 0)) * p.n_heads + head) * D + lgrp * KS);
#pragma unroll
        for (int s4 = 0; s4 < KS / 4; s4++) {
            const float4 v = qp[s4];
            qf[nt][4 * s4 + 0] = ok ? v.x * p.q_mul : 0.0f;
            qf[nt][4 * s4 + 1] = ok ? v.y * p.q_mul : 0.0f;
            qf[nt][4 * s4 + 2] = ok ? v.z * p.q_mul : 0.0f;
            qf[nt][4 * s4 + 3] = ok ? v.w * p.q_mul : 0.0f;
        }
    }

    floatx4 o[DT][NT];
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) o[t][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m[NT], lpart[NT];
    int qpos[NT], qlo[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        m[nt] = -INFINITY;
        lpart[nt] = 0.0f;
        const int lq = wq0 + nt * 16 + lrow;
        qpos[nt] = lq < q_len ? pos0 + lq : -1;  // -1: padding query, every key masked
        qlo[nt] = window_lo(pos0 + lq, p.sliding_window);
    }

    if (khi >= klo) {
        const int kfirst = (klo / KT) * KT;
        TileRegs<D, NTHR> tr;
        fetch_tile<D, NTHR, Q8>(p, b, kvh, kfirst, klo, khi, tr);
        store_tile<D, NTHR, Q8>(tr, Ks[0], Vs[0]);
        __syncthreads();
        int buf = 0;
        for (int k0 = kfirst; k0 <= khi; k0 += KT, buf ^= 1) {
            const bool more = k0 + KT <= khi;
            if (more) fetch_tile<D, NTHR, Q8>(p, b, kvh, k0 + KT, klo, khi, tr);
            const float *ks = Ks[buf];
            const float *vs = Vs[buf];

            // S^T = K . Q^T
            floatx4 sacc[2][NT];
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) sacc[mt][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s4 = 0; s4 < KS / 4; s4++) {
                float av[2][4];
#pragma unroll
                for (int mt = 0; mt < 2; mt++) {
                    const float4 a = *reinterpret_cast<const float4 *>(ks + (mt * 16 + lrow) * kRow<D> + lgrp * KS +
                                                                       4 * s4);
                    av[mt][0] = a.x;
                    av[mt][1] = a.y;
                    av[mt][2] = a.z;
                    av[mt][3] = a.w;
                }
                // the 2*NT accumulators in turn: a dependent MFMA every 2*NT issues
#pragma unroll
                for (int e = 0; e < 4; e++)
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
#pragma unroll
                        for (int nt = 0; nt < NT; nt++)
                            sacc[mt][nt] =
                                __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt][e], qf[nt][4 * s4 + e], sacc[mt][nt], 0, 0, 0);
            }

            // online softmax over this tile, per query column. Only tiles that
            // cross the diagonal, a window edge or the key range need the mask.
            const bool interior = k0 >= klo && k0 + KT - 1 <= min(khi, pos0 + wq0) &&
                                  (p.sliding_window <= 0 || k0 >= window_lo(pos0 + wq0 + QW - 1, p.sliding_window));
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                floatx4 col[2] = {sacc[0][nt], sacc[1][nt]};
                cap_and_mask<CAP>(col, p.softcap, interior, k0 + 4 * lgrp, qpos[nt], qlo[nt], klo, khi);
                sacc[0][nt] = col[0];
                sacc[1][nt] = col[1];
                float mx = -INFINITY;
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) mx = fmaxf(mx, sacc[mt][nt][i]);
                mx = max_rows4(mx);
                const float m_new = fmaxf(m[nt], mx);
                if (m_new == -INFINITY) {
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) sacc[mt][nt][i] = 0.0f;
                    continue;
                }
                const float rs = fast_exp2(m[nt] - m_new);
                m[nt] = m_new;
                float ls = 0.0f;
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float pv = fast_exp2(sacc[mt][nt][i] - m_new);
                        sacc[mt][nt][i] = pv;
                        ls += pv;
                    }
                lpart[nt] = lpart[nt] * rs + ls;
                if (__ballot(rs != 1.0f)) {  // the running max moved for some query
#pragma unroll
                    for (int t = 0; t < DT; t++) o[t][nt] *= rs;
                }
            }

            // O^T += V^T . P^T
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float *vrow = vs + (mt * 16 + 4 * lgrp + i) * kRow<D> + lrow * DT;
                    float av[DT];
#pragma unroll
                    for (int t4 = 0; t4 < DT / 4; t4++) {
                        const float4 a = reinterpret_cast<const float4 *>(vrow)[t4];
                        av[4 * t4] = a.x;
                        av[4 * t4 + 1] = a.y;
                        av[4 * t4 + 2] = a.z;
                        av[4 * t4 + 3] = a.w;
                    }
#pragma unroll
                    for (int t = 0; t < DT; t++)
#pragma unroll
                        for (int nt = 0; nt < NT; nt++)
                            o[t][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t], sacc[mt][nt][i], o[t][nt], 0, 0, 0);
                }
            }

            if (more) store_tile<D, NTHR, Q8>(tr, Ks[buf ^ 1], Vs[buf ^ 1]);
            __syncthreads();
        }
    }

    // normalise and store: lane holds O^T[d = (4*lgrp + r)*DT + t][query lrow]
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        float lt = lpart[nt];
        lt = sum_rows4(lt);
        const int lq = wq0 + nt * 16 + lrow;
        if (lq >= q_len) continue;
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        float *op = p.out + ((int64_t)(row0 + lq) * p.n_heads + head) * D + 4 * lgrp * DT;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int t4 = 0; t4 < DT / 4; t4++)
                *reinterpret_cast<float4 *>(op + r * DT + 4 * t4) =
                    make_float4(o[4 * t4][nt][r] * inv, o[4 * t4 + 1][nt][r] * inv, o[4 * t4 + 2][nt][r] * inv,
                                o[4 * t4 + 3][nt][r] * inv);
    }
}

// ---------------------------------------------------------------------------
// bf16-input variant: Q, K, V and the probabilities are rounded to bf16 and
// both products run on v_mfma_f32_16x16x32_bf16 with fp32 accumulation; the
// softmax stays fp32. Same workgroup shape, masks and online softmax as the
// fp32 kernel. K is staged row-major and V transposed (Vt[d][key]) in LDS
// as bf16, so every MFMA operand a lane needs is one 8- or 16-byte read.
//   S^T[key][q] = K . Q^T   A = K (16 keys x 32 d), B = Q^T from registers
//   O^T[d][q]  += V^T . P^T A = Vt (16 d x 32 keys), B = P^T packed from the
//                           S^T accumulators: k-slots 0..3 of lane group g
//                           are keys 4g+r of the first 16-key half and 4..7
//                           the same keys of the second half, which is what
//                           the lane's two accumulators hold.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

template <int D>
constexpr int kKRowH = D + 8;  // K row in LDS (bf16): 16 bytes of padding
constexpr int kVtRowH = KT + 8;  // Vt row in LDS (bf16): 32 keys + 16 bytes

// The 4 keys x 4 dims block of K and of V that one thread stages, as f32.
struct Block44 {
    float4 k[4];  // k[i] = K[key 4*kq + i][4*dq .. 4*dq+3]
    float4 v[4];  // v[i] = V[key 4*kq + i][4*dq .. 4*dq+3]
};

template <int D, bool Q8>
__device__ __forceinline__ void fetch_block44(const PrefillParams &p, int b, int kvh, int key0, int d0, int klo,
                                              int khi, Block44 &o) {
    const int64_t head_off = (int64_t)kvh * p.kv.head_stride;
    // key0 is a multiple of 4, so the 4 keys share one page; a block past
    // khi (zeroed below) looks up khi's page, so the page-table read stays
    // inside the sequence's row
    const int64_t pid = map_page(p.pm, b, min(key0, max(khi, 0)) >> 4);
    if constexpr (Q8) {
        const int64_t hb = pid * p.kv.page_stride + head_off;
        const int slot0 = key0 & 15;
        const int blk = d0 >> 5;
        const uint16_t *vsp = reinterpret_cast<const uint16_t *>(p.kv.vs + hb);
        const uint16_t *ksp = reinterpret_cast<const uint16_t *>(p.kv.ks + hb);
        // V: 4 consecutive slots of one d are 4 consecutive bytes (q8v_off)
        float vq[4][4];  // [d][key]
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t w = *reinterpret_cast<const uint32_t *>(p.kv.v + hb + q8v_off(slot0, d0 + j, D));
#pragma unroll
            for (int i = 0; i < 4; i++) vq[j][i] = (float)((int)((w >> (8 * i)) & 0xff) - 128);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kp = key0 + i;
            const bool ok = kp >= klo && kp <= khi;
            // K: 4 consecutive d of one slot are 4 consecutive bytes (q8k_off)
            const uint32_t w = *reinterpret_cast<const uint32_t *>(p.kv.k + hb + q8k_off(slot0 + i, d0, D));
            const float ksc = ok ? __half2float(__ushort_as_half(ksp[q8ks_off(slot0 + i, blk, D)])) : 0.0f;
            const float vsc = ok ? __half2float(__ushort_as_half(vsp[(slot0 + i) * (D / 32) + blk])) : 0.0f;
            o.k[i] = make_float4((float)((int)(w & 0xff) - 128) * ksc, (float)((int)((w >> 8) & 0xff) - 128) * ksc,
                                 (float)((int)((w >> 16) & 0xff) - 128) * ksc,
                                 (float)((int)((w >> 24) & 0xff) - 128) * ksc);
            o.v[i] = make_float4(vq[0][i] * vsc, vq[1][i] * vsc, vq[2][i] * vsc, vq[3][i] * vsc);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kp = key0 + i;
            if (kp >= klo && kp <= khi) {
                const int64_t base =
                    pid * p.kv.page_stride + head_off + (int64_t)((kp & 15)) * p.kv.row_stride + (int64_t)d0 * 4;
                o.k[i] = *reinterpret_cast<const float4 *>(p.kv.k + base);
                o.v[i] = *reinterpret_cast<const float4 *>(p.kv.v + base);
            } else {
                o.k[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                o.v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
    }
}

__device__ __forceinline__ bf16x4 to_bf16x4(float a, float b, float c, float d) {
    return bf16x4{(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
}

template <int D>
__device__ __forceinline__ void store_block44(const Block44 &o, int kq, int dq, __bf16 *Kh, __bf16 *Vt) {
#pragma unroll
    for (int i = 0; i < 4; i++)
        *reinterpret_cast<bf16x4 *>(Kh + (4 * kq + i) * kKRowH<D> + 4 * dq) =
            to_bf16x4(o.k[i].x, o.k[i].y, o.k[i].z, o.k[i].w);
    *reinterpret_cast<bf16x4 *>(Vt + (4 * dq + 0) * kVtRowH + 4 * kq) =
        to_bf16x4(o.v[0].x, o.v[1].x, o.v[2].x, o.v[3].x);
    *reinterpret_cast<bf16x4 *>(Vt + (4 * dq + 1) * kVtRowH + 4 * kq) =
        to_bf16x4(o.v[0].y, o.v[1].y, o.v[2].y, o.v[3].y);
    *reinterpret_cast<bf16x4 *>(Vt + (4 * dq + 2) * kVtRowH + 4 * kq) =
        to_bf16x4(o.v[0].z, o.v[1].z, o.v[2].z, o.v[3].z);
    *reinterpret_cast<bf16x4 *>(Vt + (4 * dq + 3) * kVtRowH + 4 * kq) =
        to_bf16x4(o.v[0].w, o.v[1].w, o.v[2].w, o.v[3].w);
}

template <int D, int NTHR>
struct TileBlocks {
    static constexpr int UNITS = (KT / 4) * (D / 4);
    static constexpr int PER_THREAD = (UNITS + NTHR - 1) / NTHR;
    Block44 blk[PER_THREAD];
};

template <int D, int NTHR, bool Q8>
__device__ __forceinline__ void fetch_tile_bf16(const PrefillParams &p, int b, int kvh, int k0, int klo, int khi,
                                                TileBlocks<D, NTHR> &t) {
#pragma unroll
    for (int j = 0; j < TileBlocks<D, NTHR>::PER_THREAD; j++) {
        const int u = threadIdx.x + j * NTHR;
        if (u >= TileBlocks<D, NTHR>::UNITS) break;
        const int kq = u / (D / 4);
        const int dq = u - kq * (D / 4);
        fetch_block44<D, Q8>(p, b, kvh, k0 + 4 * kq, 4 * dq, klo, khi, t.blk[j]);
    }
}

template <int D, int NTHR>
__device__ __forceinline__ void store_tile_bf16(const TileBlocks<D, NTHR> &t, __bf16 *Kh, __bf16 *Vt) {
#pragma unroll
    for (int j = 0; j < TileBlocks<D, NTHR>::PER_THREAD; j++) {
        const int u = threadIdx.x + j * NTHR;
        if (u >= TileBlocks<D, NTHR>::UNITS) break;
        const int kq = u / (D / 4);
        const int dq = u - kq * (D / 4);
        store_block44<D>(t.blk[j], kq, dq, Kh, Vt);
    }
}

// Waves per workgroup of the bf16 kernel (32 queries each): 8 share each
// staged K/V tile (d = 256: 4, whose registers need the 512-VGPR budget of
// one wave per SIMD).
template <int D>
constexpr int kBf16Waves = D == 256 ? 4 : 8;

// bf16 softmax: how far (log2 units) a score may pass the row's running
// maximum before the maximum, and with it O, is rescaled.
constexpr float kLazyMax = 8.0f;
// The bf16 kernels' reference maximum before a query's first attended key:
// finite, so the first attended tile is an ordinary move of the reference
// (its factor 2^(-1e30 - max) = 0 scales the still-zero O and sums) and the
// per-tile logic needs no "no key yet" case; a masked score (-inf) still
// gives p = 0, and a query that attends no key keeps l = 0 (output 0).
constexpr float kMInit = -1e30f;

// S^T accumulators of a tile before S = K.Q^T: zero (the first MFMA takes an
// inline 0), so the scores arrive absolute and p = 2^(s - m) takes one
// subtraction per score.
template <int NT>
__device__ __forceinline__ void bf16_score_init(floatx4 (&sacc)[2][NT]) {
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int mt = 0; mt < 2; mt++) sacc[mt][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
}

// max of three floats as one v_maximum3_f32 (as max2f)
__device__ __forceinline__ float max3f(float a, float b, float c) { return max2f(max2f(a, b), c); }

// Online softmax of one 32-key tile of the bf16 kernels (both share it):
// soft-cap and (MASK) the causal/window mask, the lazy maximum (the reference
// moves only when a score passes it by more than 8 log2 units, so p stays at
// most 256, exact range for bf16 and f32, and the rescale of O is rare), p =
// 2^(s - m) rounded to bf16 for both MFMAs, and the factor rs[nt] that O and
// the row sums take before this tile is added (bf16_rescale). Each lane first
// takes the maximum of its own 8 scores of a query; only when one of them
// passes its reference by more than the margin (in some lane of the wave: a
// wave-uniform branch) does the tile take the row maxima across the query's
// 4 lanes. A row whose maximum passes has that maximum in one of its lanes,
// so the rare path makes the decisions that taking every row maximum would.
template <int NT, bool CAP, bool MASK>
__device__ __forceinline__ void bf16_softmax_p(const floatx4 (&sacc)[2][NT], float (&m)[NT], float (&rs)[NT],
                                               bf16x8 (&pb)[NT], float softcap, int kbase, const int (&qpos)[NT],
                                               const int (&qlo)[NT], int klo, int khi) {
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        floatx4 col[2] = {sacc[0][nt], sacc[1][nt]};
        cap_and_mask<CAP>(col, softcap, !MASK, kbase, qpos[nt], qlo[nt], klo, khi);
        float mx = max3f(max3f(col[0][0], col[0][1], col[0][2]), max3f(col[0][3], col[1][0], col[1][1]),
                         max2f(col[1][2], col[1][3]));
        const float m_old = m[nt];
        rs[nt] = 1.0f;
        if (__ballot(mx - m_old > kLazyMax)) {
            mx = max_rows4(mx);
            // (selects: the conditions differ from lane to lane)
            const bool up = mx - m_old > kLazyMax;
            m[nt] = up ? mx : m_old;
            rs[nt] = up ? fast_exp2(m_old - mx) : 1.0f;
        }
        float pr[2][4];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) pr[mt][i] = fast_exp2(col[mt][i] - m[nt]);
        pb[nt] = bf16x8{(__bf16)pr[0][0], (__bf16)pr[0][1], (__bf16)pr[0][2], (__bf16)pr[0][3],
                        (__bf16)pr[1][0], (__bf16)pr[1][1], (__bf16)pr[1][2], (__bf16)pr[1][3]};
    }
}

// O and the row sums take the factor of a moved reference (rare: a wave-uniform
// branch per query tile).
template <int NT, int DT>
__device__ __forceinline__ void bf16_rescale(const float (&rs)[NT], floatx4 (&lacc)[NT], floatx4 (&o)[DT][NT]) {
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
        if (__ballot(rs[nt] != 1.0f)) {
#pragma unroll
            for (int t = 0; t < DT; t++) o[t][nt] *= rs[nt];
            lacc[nt] *= rs[nt];
        }
}

// The softmax of a tile inside every query's causal and window bounds, both
// query tiles decided by one wave-uniform branch: the row maxima are taken,
// and references moved, only when some lane's own maximum passes its
// reference by more than the margin; for a query tile none of whose lanes
// passes, the rare path moves nothing and scales nothing, so the decisions
// are bf16_softmax_p's.
template <int NT, int DT, bool CAP>
__device__ __forceinline__ void bf16_softmax_interior(floatx4 (&sacc)[2][NT], float (&m)[NT],
                                                      floatx4 (&lacc)[NT], floatx4 (&o)[DT][NT],
                                                      bf16x8 (&pb)[NT], float softcap) {
    float mx[NT];
    bool pass = false;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        if constexpr (CAP) {
            floatx4 col[2] = {sacc[0][nt], sacc[1][nt]};
            cap_and_mask<CAP>(col, softcap, true, 0, 0, 0, 0, 0);
            sacc[0][nt] = col[0];
            sacc[1][nt] = col[1];
        }
        mx[nt] = max3f(max3f(sacc[0][nt][0], sacc[0][nt][1], sacc[0][nt][2]),
                       max3f(sacc[0][nt][3], sacc[1][nt][0], sacc[1][nt][1]), max2f(sacc[1][nt][2], sacc[1][nt][3]));
        pass = pass || mx[nt] - m[nt] > kLazyMax;
    }
    if (__ballot(pass)) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const float mr = max_rows4(mx[nt]);
            // (selects: the conditions differ from lane to lane)
            const float m_old = m[nt];
            const bool up = mr - m_old > kLazyMax;
            m[nt] = up ? mr : m_old;
            const float rs = up ? fast_exp2(m_old - mr) : 1.0f;
            if (__ballot(rs != 1.0f)) {
#pragma unroll
                for (int t = 0; t < DT; t++) o[t][nt] *= rs;
                lacc[nt] *= rs;
            }
        }
    }
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        float pr[2][4];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) pr[mt][i] = fast_exp2(sacc[mt][nt][i] - m[nt]);
        pb[nt] = bf16x8{(__bf16)pr[0][0], (__bf16)pr[0][1], (__bf16)pr[0][2], (__bf16)pr[0][3],
                        (__bf16)pr[1][0], (__bf16)pr[1][1], (__bf16)pr[1][2], (__bf16)pr[1][3]};
    }
}

// The whole softmax of a tile whose mask need is known at run time.
template <int NT, int DT, bool CAP>
__device__ __forceinline__ void bf16_softmax(floatx4 (&sacc)[2][NT], float (&m)[NT],
                                             floatx4 (&lacc)[NT], floatx4 (&o)[DT][NT], bf16x8 (&pb)[NT],
                                             float softcap, bool interior, int kbase, const int (&qpos)[NT],
                                             const int (&qlo)[NT], int klo, int khi) {
    float rs[NT];
    if (interior)
        bf16_softmax_p<NT, CAP, false>(sacc, m, rs, pb, softcap, kbase, qpos, qlo, klo, khi);
    else
        bf16_softmax_p<NT, CAP, true>(sacc, m, rs, pb, softcap, kbase, qpos, qlo, klo, khi);
    bf16_rescale<NT, DT>(rs, lacc, o);
}

// Row sums of the tile's bf16 probabilities, from one MFMA against an
// all-ones operand: every element of a lane accumulates its query's sum.
template <int NT>
__device__ __forceinline__ void bf16_row_sums(floatx4 (&lacc)[NT], const bf16x8 (&pb)[NT]) {
    const bf16x8 ones = bf16x8{(__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f,
                               (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int nt = 0; nt < NT; nt++) lacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[nt], lacc[nt], 0, 0, 0);
}

template <int D, bool Q8, bool CAP>
__global__ __launch_bounds__(kBf16Waves<D> * 64) void prefill_bf16_kernel(const PrefillParams p) {
    constexpr int NW = kBf16Waves<D>, NT = 2, NTHR = NW * 64;
    constexpr int QW = 16 * NT;
    constexpr int KS = D / 32;  // k-steps of S (32 dims each)
    constexpr int DT = D / 16;  // d tiles of O
    __shared__ __attribute__((aligned(16))) __bf16 Kh[2][KT * kKRowH<D>];
    __shared__ __attribute__((aligned(16))) __bf16 Vt[2][D * kVtRowH];

    // grid (sequence x KV head x head group, query block): every unit's
    // longest (last) query block is dispatched before any shorter one, so the
    // grid ends on short workgroups
    const int n_hgrp = p.group / p.hpw;
    const int unit = blockIdx.x;
    const int b = unit / (p.n_kv_heads * n_hgrp);
    const int kvh = (unit - b * p.n_kv_heads * n_hgrp) / n_hgrp;
    const int hgrp = unit - (b * p.n_kv_heads + kvh) * n_hgrp;
    const int qblk = p.n_qblocks - 1 - (int)blockIdx.y;
    const int waves_per_head = NW / p.hpw;
    const int qwg = QW * waves_per_head;

    const int row0 = p.q_start[b];
    const int q_len = min(max(p.q_start[b + 1] - row0, 0), p.max_q_len);
    const int pos0 = p.pos_offset[b];
    const int qb0 = qblk * qwg;
    if (qb0 >= q_len) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lrow = lane & 15;
    const int lgrp = lane >> 4;
    const int head = kvh * p.group + hgrp * p.hpw + (wave % p.hpw);
    const int wq0 = qb0 + (wave / p.hpw) * QW;

    const int q_last = min(q_len, qb0 + qwg) - 1;
    const int khi = min(pos0 + q_last, p.pm.pos_limit - 1);
    const int klo = window_lo(pos0 + qb0, p.sliding_window);

    // Q^T operand: qb[nt][ks] = Q[query nt*16 + lrow][d = ks*32 + lgrp*8 + 0..7] as bf16
    bf16x8 qb[NT][KS];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int lq = wq0 + nt * 16 + lrow;
        const bool ok = lq < q_len;
        const float *qp = p.q + ((int64_t)(row0 + (ok ? lq : 0)) * p.n_heads + head) * D;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const float4 a = *reinterpret_cast<const float4 *>(qp + ks * 32 + lgrp * 8);
            const float4 c = *reinterpret_cast<const float4 *>(qp + ks * 32 + lgrp * 8 + 4);
            const float mul = ok ? p.q_mul : 0.0f;
            qb[nt][ks] = bf16x8{(__bf16)(a.x * mul), (__bf16)(a.y * mul), (__bf16)(a.z * mul), (__bf16)(a.w * mul),
                                (__bf16)(c.x * mul), (__bf16)(c.y * mul), (__bf16)(c.z * mul), (__bf16)(c.w * mul)};
        }
    }

    floatx4 o[DT][NT];
    floatx4 lacc[NT];
    float m[NT];  // the query's reference maximum (log2 domain)
    int qpos[NT], qlo[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
#pragma unroll
        for (int t = 0; t < DT; t++) o[t][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        lacc[nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        m[nt] = kMInit;
        const int lq = wq0 + nt * 16 + lrow;
        qpos[nt] = lq < q_len ? pos0 + lq : -1;
        qlo[nt] = window_lo(pos0 + lq, p.sliding_window);
    }
    // keys this wave's queries attend: [wlo, whi]
    const int whi = min(khi, pos0 + wq0 + QW - 1);
    const int wlo = max(klo, window_lo(pos0 + wq0, p.sliding_window));

    if (khi >= klo) {
        const int kfirst = (klo / KT) * KT;
        TileBlocks<D, NTHR> tb;
        fetch_tile_bf16<D, NTHR, Q8>(p, b, kvh, kfirst, klo, khi, tb);
        store_tile_bf16<D, NTHR>(tb, Kh[0], Vt[0]);
        __syncthreads();
        int buf = 0;
        for (int k0 = kfirst; k0 <= khi; k0 += KT, buf ^= 1) {
            const bool more = k0 + KT <= khi;
            if (more) fetch_tile_bf16<D, NTHR, Q8>(p, b, kvh, k0 + KT, klo, khi, tb);
            const __bf16 *kh = Kh[buf];
            const __bf16 *vt = Vt[buf];
            // a tile wholly past this wave's last query or before its window adds nothing
            if (k0 <= whi && k0 + KT - 1 >= wlo) {
            // S^T = K . Q^T
            floatx4 sacc[2][NT];
            bf16_score_init<NT>(sacc);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                bf16x8 a[2];
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
                    a[mt] = *reinterpret_cast<const bf16x8 *>(kh + (mt * 16 + lrow) * kKRowH<D> + ks * 32 + lgrp * 8);
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
                        sacc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt], qb[nt][ks], sacc[mt][nt], 0, 0, 0);
            }

            const bool interior = k0 >= klo && k0 + KT - 1 <= min(khi, pos0 + wq0) &&
                                  (p.sliding_window <= 0 || k0 >= window_lo(pos0 + wq0 + QW - 1, p.sliding_window));
            bf16x8 pb[NT];
            bf16_softmax<NT, DT, CAP>(sacc, m, lacc, o, pb, p.softcap, interior, k0 + 4 * lgrp, qpos, qlo, klo,
                                      khi);

            // O^T += V^T . P^T, and the row sums
            bf16_row_sums<NT>(lacc, pb);
#pragma unroll
            for (int t = 0; t < DT; t++) {
                const __bf16 *vr = vt + (16 * t + lrow) * kVtRowH;
                const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(vr + 4 * lgrp);
                const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(vr + 16 + 4 * lgrp);
                const bf16x8 a = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    o[t][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[nt], o[t][nt], 0, 0, 0);
            }
            }

            if (more) store_tile_bf16<D, NTHR>(tb, Kh[buf ^ 1], Vt[buf ^ 1]);
            __syncthreads();
        }
    }

    // normalise and store: lane holds O^T[d = 16t + 4*lgrp + r][query lrow]
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const float lt = lacc[nt][0];
        const int lq = wq0 + nt * 16 + lrow;
        if (lq >= q_len) continue;
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        float *op = p.out + ((int64_t)(row0 + lq) * p.n_heads + head) * D;
#pragma unroll
        for (int t = 0; t < DT; t++) {
            const floatx4 v = o[t][nt] * inv;
            *reinterpret_cast<float4 *>(op + 16 * t + 4 * lgrp) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
}

// ---------------------------------------------------------------------------
// Staged bf16 path: a pre-pass converts each (sequence, KV head, 32-key tile)
// the prefill reads to bf16 once, in the exact LDS image the MFMA operand
// reads want, and the main kernel copies tile images into an LDS ring with
// direct global->LDS loads (no registers, no conversion, kRingTiles - 1 tiles
// ahead).
// The image of a tile is 128*D bytes, 16-byte pieces:
//   K: piece ((mt*(D/8) + c)*16 + r) = K[key mt*16 + r][dims 8c .. 8c+7]
//   V: piece ((t*4 + g)*16 + r)      = V[keys 4g..4g+3, 16+4g..16+4g+3][dim 16t + r]
// so the 16 lanes of each read pass (r = 0..15) take 16 consecutive pieces
// of one 256-byte line: no LDS bank conflicts, and the whole image is one
// contiguous copy. Keys outside the sequence's window union [window_lo(pos0),
// last query] are zero, as the in-kernel staging zeroes them.
// Tile images in a workgroup's ring: three (48 KB at d = 128) lets three
// workgroups share a CU, so one's prologue, epilogue and barrier waits meet
// the others' matrix work; d = 256 keeps four (one workgroup per CU).
template <int D>
constexpr int kRingTiles = D == 256 ? 4 : 3;

template <int D>
constexpr int kTileImage = 128 * D;

template <int D, bool Q8>
__global__ __launch_bounds__(256) void stage_bf16_kernel(const PrefillParams p, uint8_t *img, int n_tiles) {
    const int t = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int row0 = p.q_start[b];
    const int q_len = min(max(p.q_start[b + 1] - row0, 0), p.max_q_len);
    if (q_len == 0) return;
    const int pos0 = p.pos_offset[b];
    const int khi = min(pos0 + q_len - 1, p.pm.pos_limit - 1);
    const int klo = window_lo(pos0, p.sliding_window);
    const int k0 = t * KT;
    if (khi < klo || k0 > khi || k0 + KT - 1 < klo) return;  // a tile no query of the sequence reads

    uint8_t *dst = img + (((int64_t)b * p.n_kv_heads + kvh) * n_tiles + t) * kTileImage<D>;
    constexpr int NP = 4 * D;  // pieces of K (and of V) per tile
    if constexpr (!Q8) {
        // f32 cache: a K piece is 8 consecutive dims of one key, read and
        // converted straight from the row; V pieces run across keys, so V
        // goes through LDS as bf16 rows. The tile's 32 keys lie in two pages.
        __shared__ __attribute__((aligned(16))) __bf16 Vh[KT][D + 8];
        const int64_t head_off = (int64_t)kvh * p.kv.head_stride;
        const int64_t pid0 = map_page(p.pm, b, min(k0, khi) >> 4);
        const int64_t pid1 = map_page(p.pm, b, min(k0 + 16, khi) >> 4);
        // every load of the thread is issued before any store (the stores to
        // the image could alias the cache for the compiler)
        constexpr int NV = KT * (D / 8) / 256;  // V (key, 8 dims) runs per thread
        constexpr int NK = NP / 256;            // K pieces per thread
        float4 va[NV][2], ka[NK][2];
#pragma unroll
        for (int r = 0; r < NV; r++) {
            const int u = threadIdx.x + 256 * r;
            const int key = u / (D / 8);
            const int kp = k0 + key;
            va[r][0] = va[r][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (kp >= klo && kp <= khi) {
                const float *vr = reinterpret_cast<const float *>(
                    p.kv.v + (key < 16 ? pid0 : pid1) * p.kv.page_stride + head_off +
                    (int64_t)(kp & 15) * p.kv.row_stride) + 8 * (u - key * (D / 8));
                va[r][0] = *reinterpret_cast<const float4 *>(vr);
                va[r][1] = *reinterpret_cast<const float4 *>(vr + 4);
            }
        }
#pragma unroll
        for (int r = 0; r < NK; r++) {
            const int i = threadIdx.x + 256 * r;
            const int mt = i / (D / 8 * 16);
            const int rem = i - mt * (D / 8 * 16);
            const int key = mt * 16 + (rem & 15);
            const int kp = k0 + key;
            ka[r][0] = ka[r][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (kp >= klo && kp <= khi) {
                const float *kr = reinterpret_cast<const float *>(
                    p.kv.k + (key < 16 ? pid0 : pid1) * p.kv.page_stride + head_off +
                    (int64_t)(kp & 15) * p.kv.row_stride) + 8 * (rem >> 4);
                ka[r][0] = *reinterpret_cast<const float4 *>(kr);
                ka[r][1] = *reinterpret_cast<const float4 *>(kr + 4);
            }
        }
#pragma unroll
        for (int r = 0; r < NV; r++) {
            const int u = threadIdx.x + 256 * r;
            const int key = u / (D / 8);
            const float4 x = va[r][0], y = va[r][1];
            *reinterpret_cast<bf16x8 *>(&Vh[key][8 * (u - key * (D / 8))]) =
                bf16x8{(__bf16)x.x, (__bf16)x.y, (__bf16)x.z, (__bf16)x.w,
                       (__bf16)y.x, (__bf16)y.y, (__bf16)y.z, (__bf16)y.w};
        }
        // K pieces, straight to the image
#pragma unroll
        for (int r = 0; r < NK; r++) {
            const float4 x = ka[r][0], y = ka[r][1];
            *reinterpret_cast<bf16x8 *>(dst + (int64_t)(threadIdx.x + 256 * r) * 16) =
                bf16x8{(__bf16)x.x, (__bf16)x.y, (__bf16)x.z, (__bf16)x.w,
                       (__bf16)y.x, (__bf16)y.y, (__bf16)y.z, (__bf16)y.w};
        }
        __syncthreads();
        for (int i = threadIdx.x; i < NP; i += 256) {
            const int tt = i >> 6;
            const int g = (i >> 4) & 3;
            const int d = 16 * tt + (i & 15);
            const bf16x8 h = bf16x8{Vh[4 * g][d], Vh[4 * g + 1][d], Vh[4 * g + 2][d], Vh[4 * g + 3][d],
                                    Vh[16 + 4 * g][d], Vh[17 + 4 * g][d], Vh[18 + 4 * g][d], Vh[19 + 4 * g][d]};
            *reinterpret_cast<bf16x8 *>(dst + 64 * D + (int64_t)i * 16) = h;
        }
        return;
    }
    __shared__ __attribute__((aligned(16))) float Kf[KT][D + 4];
    __shared__ __attribute__((aligned(16))) float Vf[KT][D + 4];
    for (int u = threadIdx.x; u < (KT / 4) * (D / 4); u += 256) {
        const int kq = u / (D / 4);
        const int dq = u - kq * (D / 4);
        Block44 blk;
        fetch_block44<D, Q8>(p, b, kvh, k0 + 4 * kq, 4 * dq, klo, khi, blk);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *reinterpret_cast<float4 *>(&Kf[4 * kq + i][4 * dq]) = blk.k[i];
            *reinterpret_cast<float4 *>(&Vf[4 * kq + i][4 * dq]) = blk.v[i];
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < NP; i += 256) {
        const int mt = i / (D / 8 * 16);
        const int rem = i - mt * (D / 8 * 16);
        const int c = rem >> 4;
        const int key = mt * 16 + (rem & 15);
        const float *kr = &Kf[key][8 * c];
        const bf16x8 h = bf16x8{(__bf16)kr[0], (__bf16)kr[1], (__bf16)kr[2], (__bf16)kr[3],
                                (__bf16)kr[4], (__bf16)kr[5], (__bf16)kr[6], (__bf16)kr[7]};
        *reinterpret_cast<bf16x8 *>(dst + (int64_t)i * 16) = h;
    }
    for (int i = threadIdx.x; i < NP; i += 256) {
        const int tt = i >> 6;
        const int g = (i >> 4) & 3;
        const int d = 16 * tt + (i & 15);
        const bf16x8 h = bf16x8{(__bf16)Vf[4 * g][d], (__bf16)Vf[4 * g + 1][d], (__bf16)Vf[4 * g + 2][d],
                                (__bf16)Vf[4 * g + 3][d], (__bf16)Vf[16 + 4 * g][d], (__bf16)Vf[17 + 4 * g][d],
                                (__bf16)Vf[18 + 4 * g][d], (__bf16)Vf[19 + 4 * g][d]};
        *reinterpret_cast<bf16x8 *>(dst + 64 * D + (int64_t)i * 16) = h;
    }
}

// 16 bytes per lane from sbase + voff into LDS at m0 + 16*lane (m0 restored).
// Default (cached) loads: each tile image is read by every query block of
// its unit. The s_nop is the wait state an LDS-DMA load needs after an SALU
// write of M0, which the compiler cannot insert into inline assembly.
__device__ __forceinline__ void lds_copy16(const uint8_t *sbase, uint32_t voff, uint32_t m0) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(voff), "s"(sbase), "s"(m0)
        : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waves per workgroup of the staged kernel (32 queries each): one per SIMD;
// a CU holds several workgroups.
template <int D>
constexpr int kBf16sWaves = 4;
// Kilobyte copies per wave of the staged kernel's tile ring (every wave copies).
template <int D>
constexpr int kCopiesPerWave = D == 64 ? 2 : (D == 128 ? 4 : 8);
// Waves per SIMD the staged kernel's registers are sized for: d = 64: 4
// (<= 128 VGPRs), d = 128: 3 (<= 168; the soft-capped variant spills one
// register), d = 256: 1.
template <int D>
constexpr int kBf16sOccupancy = D == 64 ? 4 : (D == 128 ? 3 : 1);

template <int D, bool CAP>
__global__ __launch_bounds__(kBf16sWaves<D> * 64, kBf16sOccupancy<D>) void prefill_bf16s_kernel(const PrefillParams p,
                                                                          const uint8_t *img, int n_tiles) {
    constexpr int NW = kBf16sWaves<D>, NT = 2;
    constexpr int QW = 16 * NT;
    constexpr int KS = D / 32;
    constexpr int DT = D / 16;
    constexpr int NC = kTileImage<D> / 1024;  // 1 KB copies per tile, dealt to the waves in turn
    constexpr int RT = kRingTiles<D>;
    __shared__ __attribute__((aligned(16))) uint8_t ring[RT][kTileImage<D>];

    const int n_hgrp = p.group / p.hpw;
    const int unit = blockIdx.x;
    const int b = unit / (p.n_kv_heads * n_hgrp);
    const int kvh = (unit - b * p.n_kv_heads * n_hgrp) / n_hgrp;
    const int hgrp = unit - (b * p.n_kv_heads + kvh) * n_hgrp;
    const int qblk = p.n_qblocks - 1 - (int)blockIdx.y;
    const int waves_per_head = NW / p.hpw;
    const int qwg = QW * waves_per_head;

    const int row0 = p.q_start[b];
    const int q_len = min(max(p.q_start[b + 1] - row0, 0), p.max_q_len);
    const int pos0 = p.pos_offset[b];
    const int qb0 = qblk * qwg;
    if (qb0 >= q_len) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 15;
    const int lgrp = lane >> 4;
    const int head = kvh * p.group + hgrp * p.hpw + (wave % p.hpw);
    const int wq0 = qb0 + (wave / p.hpw) * QW;

    const int q_last = min(q_len, qb0 + qwg) - 1;
    const int khi = min(pos0 + q_last, p.pm.pos_limit - 1);
    const int klo = window_lo(pos0 + qb0, p.sliding_window);

    bf16x8 qb[NT][KS];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int lq = wq0 + nt * 16 + lrow;
        const bool ok = lq < q_len;
        const float *qp = p.q + ((int64_t)(row0 + (ok ? lq : 0)) * p.n_heads + head) * D;
        // q rows are read once per call and the output rows written once:
        // non-temporal accesses (measured: the f32 output stream otherwise
        // slows the q reads of the workgroups starting beside it)
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const floatx4 a = __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(qp + ks * 32 + lgrp * 8));
            const floatx4 c = __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(qp + ks * 32 + lgrp * 8 + 4));
            const float mul = ok ? p.q_mul : 0.0f;
            qb[nt][ks] = bf16x8{(__bf16)(a.x * mul), (__bf16)(a.y * mul), (__bf16)(a.z * mul), (__bf16)(a.w * mul),
                                (__bf16)(c.x * mul), (__bf16)(c.y * mul), (__bf16)(c.z * mul), (__bf16)(c.w * mul)};
        }
    }

    floatx4 o[DT][NT];
    floatx4 lacc[NT];
    float m[NT];
    int qpos[NT], qlo[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
#pragma unroll
        for (int t = 0; t < DT; t++) o[t][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        lacc[nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        m[nt] = kMInit;
        const int lq = wq0 + nt * 16 + lrow;
        qpos[nt] = lq < q_len ? pos0 + lq : -1;
        qlo[nt] = window_lo(pos0 + lq, p.sliding_window);
    }
    // keys this wave's queries attend: [wlo, whi]
    const int whi = min(khi, pos0 + wq0 + QW - 1);
    const int wlo = max(klo, window_lo(pos0 + wq0, p.sliding_window));

    if (khi >= klo) {
        const int tfirst = klo / KT;
        const int n = khi / KT - tfirst + 1;
        const uint8_t *unit_img = img + ((int64_t)b * p.n_kv_heads + kvh) * n_tiles * kTileImage<D>;
        const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(
            (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)&ring[0][0]);
        // A tile's NC kilobyte copies go to the first NC / CPW waves, CPW each,
        // so every wave that copies has the same count in flight and one
        // wait count (chosen by the tiles left) serves every wave.
        constexpr int CPW = kCopiesPerWave<D>;
        static_assert(NC % CPW == 0 && NC / CPW <= NW, "copies cover the tile");
        auto issue = [&](int i) {
            if (wave < NC / CPW) {
                const uint8_t *src = unit_img + (int64_t)(tfirst + i) * kTileImage<D>;
                const uint32_t dst = ring_lds + (uint32_t)((i % RT) * kTileImage<D>);
#pragma unroll
                for (int c = 0; c < CPW; c++) {
                    const int piece = wave * CPW + c;
                    lds_copy16(src, (uint32_t)(piece * 1024 + lane * 16), dst + piece * 1024);
                }
            }
        };
#pragma unroll
        for (int i = 0; i < RT - 1; i++)
            if (i < n) issue(i);
        static_assert(RT == 3 || RT == 4, "the waits below assume one or two tiles in flight behind the current one");
        // this wave's copies of tile i have landed (later tiles may be in
        // flight), and every wave's have; every wave is also done with tile
        // i - 1, whose buffer the next copy reuses
        auto arrive = [&](int i) {
            const int ahead = n - 1 - i;
            if (RT == 4 && ahead >= 2)
                wait_vm<(RT - 2) * CPW>();
            else if (ahead >= 1)
                wait_vm<CPW>();
            else
                wait_vm<0>();
            __syncthreads();
            if (i + RT - 1 < n) issue(i + RT - 1);
        };
        // S^T = K . Q^T of tile i
        auto scores = [&](const uint8_t *kimg, floatx4 (&sacc)[2][NT]) {
            bf16_score_init<NT>(sacc);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                bf16x8 a[2];
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
                    a[mt] = *reinterpret_cast<const bf16x8 *>(kimg + ((mt * (D / 8) + ks * 4 + lgrp) * 16 + lrow) * 16);
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
                        sacc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt], qb[nt][ks], sacc[mt][nt], 0, 0, 0);
            }
        };
        // O^T += V^T . P^T, and the row sums
        auto accumulate = [&](const uint8_t *vimg, const bf16x8 (&pb)[NT]) {
            bf16_row_sums<NT>(lacc, pb);
#pragma unroll
            for (int t = 0; t < DT; t++) {
                const bf16x8 a = *reinterpret_cast<const bf16x8 *>(vimg + ((t * 4 + lgrp) * 16 + lrow) * 16);
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    o[t][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[nt], o[t][nt], 0, 0, 0);
            }
        };
        // The leading tiles inside the causal and window bounds of every query
        // of the workgroup, when its waves share one query block (one q-head
        // each): no mask, no skip test and one lazy-maximum branch per tile.
        int n_int = 0;
        if (p.hpw == NW) {
            const int k_first = tfirst * KT;
            const bool lead = k_first >= klo &&
                              (p.sliding_window <= 0 || k_first >= window_lo(pos0 + wq0 + QW - 1, p.sliding_window));
            if (lead) n_int = max(0, min(n, (min(khi, pos0 + wq0) + 1) / KT - tfirst));
        }
        int i = 0;
        for (; i < n_int; i++) {
            arrive(i);
            const uint8_t *kimg = ring[i % RT];
            floatx4 sacc[2][NT];
            scores(kimg, sacc);
            bf16x8 pb[NT];
            bf16_softmax_interior<NT, DT, CAP>(sacc, m, lacc, o, pb, p.softcap);
            accumulate(kimg + 64 * D, pb);
        }
        for (; i < n; i++) {
            arrive(i);
            const int k0 = (tfirst + i) * KT;
            // a tile wholly past this wave's last query (the causal diagonal of
            // the workgroup's later waves) or before its window adds nothing
            if (k0 > whi || k0 + KT - 1 < wlo) continue;
            const uint8_t *kimg = ring[i % RT];
            floatx4 sacc[2][NT];
            scores(kimg, sacc);
            const bool interior = k0 >= klo && k0 + KT - 1 <= min(khi, pos0 + wq0) &&
                                  (p.sliding_window <= 0 || k0 >= window_lo(pos0 + wq0 + QW - 1, p.sliding_window));
            bf16x8 pb[NT];
            bf16_softmax<NT, DT, CAP>(sacc, m, lacc, o, pb, p.softcap, interior, k0 + 4 * lgrp, qpos, qlo, klo,
                                      khi);
            accumulate(kimg + 64 * D, pb);
        }
    }

    // Output rows through LDS (the ring is free once every wave is done with
    // it): a lane holds 4 dims of one query, so direct stores would write
    // half lines; read back row-major, each store instruction writes whole
    // D-float rows. Each wave stages its 16 queries of one nt at a time in
    // its own region (rows padded by 4 floats against bank conflicts); a
    // wave's LDS operations run in order, so it needs no barrier of its own.
    constexpr int SROW = D + 4;
    static_assert(NW * 16 * SROW * 4 <= kRingTiles<D> * kTileImage<D>, "output staging fits the ring");
    __syncthreads();
    float *stage = reinterpret_cast<float *>(&ring[0][0]) + wave * 16 * SROW;
    constexpr int LPR = D / 4;    // lanes per row (16 bytes each)
    constexpr int RPI = 64 / LPR;  // rows per store instruction
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const float lt = lacc[nt][0];
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
        for (int t = 0; t < DT; t++)
            *reinterpret_cast<floatx4 *>(stage + lrow * SROW + 16 * t + 4 * lgrp) = o[t][nt] * inv;
#pragma unroll
        for (int k = 0; k < 16 / RPI; k++) {
            const int r = k * RPI + lane / LPR;
            const int c = (lane % LPR) * 4;
            const floatx4 v = *reinterpret_cast<const floatx4 *>(stage + r * SROW + c);
            const int lq = wq0 + nt * 16 + r;
            if (lq < q_len)
                __builtin_nontemporal_store(v, reinterpret_cast<floatx4 *>(p.out + ((int64_t)(row0 + lq) * p.n_heads + head) * D + c));
        }
    }
}

// The staged path's launches; GLA_ERR_* when a launch fails.
template <int D, bool Q8>
int launch_bf16_staged(gla_ctx *ctx, const PrefillParams &prm, dim3 grid, int n_seqs, uint8_t *img, int n_tiles) {
    hipLaunchKernelGGL((stage_bf16_kernel<D, Q8>), dim3(n_tiles, prm.n_kv_heads, n_seqs), dim3(256), 0, ctx->stream,
                       prm, img, n_tiles);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "stage_bf16_kernel launch: %s", hipGetErrorString(e));
    if (prm.softcap > 0.0f)
        hipLaunchKernelGGL((prefill_bf16s_kernel<D, true>), grid, dim3(kBf16sWaves<D> * 64), 0, ctx->stream, prm,
                           (const uint8_t *)img, n_tiles);
    else
        hipLaunchKernelGGL((prefill_bf16s_kernel<D, false>), grid, dim3(kBf16sWaves<D> * 64), 0, ctx->stream, prm,
                           (const uint8_t *)img, n_tiles);
    e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "prefill_bf16s_kernel launch: %s", hipGetErrorString(e));
    return GLA_OK;
}

template <int D, bool Q8>
int launch_bf16(gla_ctx *ctx, const PrefillParams &prm, dim3 grid) {
    if (prm.softcap > 0.0f)
        hipLaunchKernelGGL((prefill_bf16_kernel<D, Q8, true>), grid, dim3(kBf16Waves<D> * 64), 0, ctx->stream, prm);
    else
        hipLaunchKernelGGL((prefill_bf16_kernel<D, Q8, false>), grid, dim3(kBf16Waves<D> * 64), 0, ctx->stream, prm);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "prefill_bf16_kernel launch: %s", hipGetErrorString(e));
    return GLA_OK;
}

template <int D, int NT, int NW, bool Q8>
int launch_f32(gla_ctx *ctx, const PrefillParams &prm, dim3 grid) {
    if (prm.softcap > 0.0f)
        hipLaunchKernelGGL((prefill_f32_kernel<D, NT, NW, Q8, true>), grid, dim3(NW * 64), 0, ctx->stream, prm);
    else
        hipLaunchKernelGGL((prefill_f32_kernel<D, NT, NW, Q8, false>), grid, dim3(NW * 64), 0, ctx->stream, prm);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "prefill_f32_kernel launch: %s", hipGetErrorString(e));
    return GLA_OK;
}

// Shapes per head_dim: queries per wave (16*NT) and waves per workgroup.
// d128 (cfg4): 4 waves of 32 queries. 8 waves of 16 queries (4 waves per
// SIMD instead of 2) measured 4% slower: each K/V operand read from LDS then
// feeds one MFMA instead of two.
template <int D>
struct PrefillShape;
template <>
struct PrefillShape<64> {
    static constexpr int NT = 2, NW = 4;
};
template <>
struct PrefillShape<128> {
    static constexpr int NT = 2, NW = 4;
};
template <>
struct PrefillShape<256> {
    static constexpr int NT = 1, NW = 4;
};

template <int D>
int launch_shape(gla_ctx *ctx, bool q8, const PrefillParams &prm, dim3 grid) {
    using S = PrefillShape<D>;
    return q8 ? launch_f32<D, S::NT, S::NW, true>(ctx, prm, grid) : launch_f32<D, S::NT, S::NW, false>(ctx, prm, grid);
}

}  // namespace

int launch_prefill(gla_ctx *ctx, const PrefillLaunch &a) {
    const int D = a.head_dim;
    const int group = a.n_heads / a.n_kv_heads;
    const int hpw = (group % 4 == 0) ? 4 : ((group % 2 == 0) ? 2 : 1);
    int NT = 1, NW = 4;
    switch (D) {
    case 64:
        NT = PrefillShape<64>::NT, NW = PrefillShape<64>::NW;
        break;
    case 128:
        NT = PrefillShape<128>::NT, NW = PrefillShape<128>::NW;
        break;
    case 256:
        NT = PrefillShape<256>::NT, NW = PrefillShape<256>::NW;
        break;
    default:
        return set_error(GLA_ERR_INVALID, "unsupported head_dim %d", D);
    }
    // bf16: the staged path keeps the bf16 tile images of every (sequence, KV
    // head) in scratch, up to 1 GiB, and its staging grid has one z row per
    // sequence (at most 65,535); beyond either each workgroup converts its own
    // tiles (prefill_bf16_kernel, the same bits)
    const int n_tiles = (a.pm.pos_limit + KT - 1) / KT;
    const size_t img_bytes = (size_t)a.n_seqs * a.n_kv_heads * (size_t)n_tiles * (size_t)(128 * D);
    const bool staged = a.precision == GLA_PREC_BF16 && getenv("GLA_BF16_UNSTAGED") == nullptr && n_tiles > 0 &&
                        img_bytes <= ((size_t)1 << 30) && a.n_seqs <= 65535;
    if (a.precision == GLA_PREC_BF16) {
        NT = 2;
        if (staged)
            NW = D == 64 ? kBf16sWaves<64> : (D == 128 ? kBf16sWaves<128> : kBf16sWaves<256>);
        else
            NW = D == 256 ? kBf16Waves<256> : kBf16Waves<128>;
    }
    const int qwg = 16 * NT * (NW / hpw);
    PrefillParams prm;
    prm.kv = a.kv;
    prm.pm = a.pm;
    prm.q_start = a.q_start;
    prm.pos_offset = a.pos_offset;
    prm.q = a.q;
    prm.out = a.out;
    prm.n_heads = a.n_heads;
    prm.n_kv_heads = a.n_kv_heads;
    prm.group = group;
    prm.hpw = hpw;
    prm.n_qblocks = (a.max_q_len + qwg - 1) / qwg;
    prm.max_q_len = a.max_q_len;
    const bool cap = a.softcap > 0.0f;
    prm.q_mul = cap ? a.scale : a.scale * kLog2e;
    prm.softcap = cap ? a.softcap : 0.0f;
    prm.sliding_window = a.sliding_window;
    if (prm.n_qblocks > 65535) return set_error(GLA_ERR_INVALID, "prefill: %d query blocks > 65535", prm.n_qblocks);
    dim3 grid(a.n_seqs * a.n_kv_heads * (group / hpw), prm.n_qblocks, 1);
    if (a.precision == GLA_PREC_BF16) {
        if (staged) {
            void *scr = nullptr;
            int rc = ensure_scratch(ctx, img_bytes, &scr);
            if (rc != GLA_OK) return rc;
            uint8_t *img = (uint8_t *)scr;
            switch (D) {
            case 64:
                return a.q8 ? launch_bf16_staged<64, true>(ctx, prm, grid, a.n_seqs, img, n_tiles)
                            : launch_bf16_staged<64, false>(ctx, prm, grid, a.n_seqs, img, n_tiles);
            case 128:
                return a.q8 ? launch_bf16_staged<128, true>(ctx, prm, grid, a.n_seqs, img, n_tiles)
                            : launch_bf16_staged<128, false>(ctx, prm, grid, a.n_seqs, img, n_tiles);
            default:
                return a.q8 ? launch_bf16_staged<256, true>(ctx, prm, grid, a.n_seqs, img, n_tiles)
                            : launch_bf16_staged<256, false>(ctx, prm, grid, a.n_seqs, img, n_tiles);
            }
        }
        switch (D) {
        case 64:
            return a.q8 ? launch_bf16<64, true>(ctx, prm, grid) : launch_bf16<64, false>(ctx, prm, grid);
        case 128:
            return a.q8 ? launch_bf16<128, true>(ctx, prm, grid) : launch_bf16<128, false>(ctx, prm, grid);
        default:
            return a.q8 ? launch_bf16<256, true>(ctx, prm, grid) : launch_bf16<256, false>(ctx, prm, grid);
        }
    }
    switch (D) {
    case 64:
        return launch_shape<64>(ctx, a.q8, prm, grid);
    case 128:
        return launch_shape<128>(ctx, a.q8, prm, grid);
    default:
        return launch_shape<256>(ctx, a.q8, prm, grid);
    }
}

}  // namespace gla
