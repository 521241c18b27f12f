// gla_ops.hip -- the GPU ops beside attention on a decode step: RoPE on q/k
// and the Q8_0 weight matvec of the Q/K/V/O projections, so the step stays
// on the device between the projections and attention.
//
//   gla_rope          ops::rope                         src/tensor/ops.rs:212-245
//   gla_q8w_create    GpuBackend::upload_buffer of GGML Q8_0 weights
//                                                       src/backend/gpu.rs:111-121
//   gla_matvec_q8_0   QuantizedTensor::matvec / matvec_batch over Q8_0,
//                     matvec_q8_0.wgsl               src/tensor/quantized.rs:247-346, :587-610
//
// Matvec design. GGML's 34-byte blocks ([f16 scale][32 x i8]) are not 16-byte
// aligned, so the weights are repacked once, on upload, into the operand
// order of v_mfma_f32_16x16x32_f16: a row tile of 16 rows and a pair of
// 32-element blocks is one 16-byte piece per lane (lane l: row l%16, elements
// (l/16)*8 .. +8 of each block, stored as x + 128 so that one v_perm makes
// the exact f16 of 1024 + byte), and the pair's 32 scales are one 16-byte
// read per lane. The activations are split per call into two f16 pieces
// (hi = f16(x * 2^s), lo = f16(x * 2^s - hi), s per vector and K slice
// putting the slice's largest |x| near 2^14), so each block's product runs as two MFMAs with
// exact int8 x f16 products and f32 accumulation; the f16 block scale is
// applied in f32 per block, as the reference applies it. Each launch covers
// up to 64 vectors, so the weights are read once per 64 vectors; K is split
// across workgroups (the slices summed in order by each row group's last
// workgroup to finish) so that each CU reads only its slice of the
// activation pieces. Up to four vectors
// take the vector-ALU kernel instead (x in f32 from LDS, no pieces). Bound:
// HBM on the weights (34 bytes per 32 weights).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "gla_internal.h"

struct gla_q8w {
    gla_ctx *ctx = nullptr;
    int rows = 0;
    int cols = 0;
    int n_tiles = 0;  // ceil(rows / 16)
    int n_pairs = 0;  // ceil(cols / 64)
    uint8_t *quants = nullptr;  // [n_tiles][n_pairs][64 lanes][16 B]
    uint16_t *scales = nullptr;  // [n_tiles][n_pairs][16 rows][2 blocks] f16
};

namespace gla {

void detach_q8w(gla_q8w *w) {
    if (w->quants) (void)hipFree(w->quants);
    if (w->scales) (void)hipFree(w->scales);
    w->quants = nullptr;
    w->scales = nullptr;
    w->ctx = nullptr;
}

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---- RoPE -----------------------------------------------------------------

// The frequencies of up to kRopeLaunchPairs pairs, passed by value (1 KiB of
// kernel arguments: no device buffer, nothing to copy before the launch).
constexpr int kRopeLaunchPairs = 256;
struct RopeFreqs {
    float f[kRopeLaunchPairs];
};

// One thread per (row, head, pair) of the launch's pairs p0 .. p0 + n_pairs:
// the pair (i, i+1), i = 2 * pair, rotated by (pos / scaling) * freq, with
// the reference's f32 operations in its order and no contraction. freq =
// 1 / powf(base, i / d) comes from the host's powf, the libm routine the
// reference's f32::powf calls, because that powf is not correctly rounded for
// every argument (a device pow rounded to f32 differs from it in about one
// case in a thousand, and the angle then differs by an ulp times pos).
__global__ __launch_bounds__(256) void rope_kernel(float *x, int n_rows, int n_heads, int head_dim, int p0,
                                                   int n_pairs, const int32_t *pos, float scaling_factor,
                                                   RopeFreqs fr) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)n_rows * n_heads * n_pairs;
    if (t >= total) return;
    const int pr = (int)(t % n_pairs);
    const int64_t rh = t / n_pairs;
    const int row = (int)(rh / n_heads);
    const int i = 2 * (p0 + pr);
    const float pos_scaled = (float)pos[row] / scaling_factor;
    const float freq = fr.f[pr];
    const float angle = pos_scaled * freq;
    const float c = cosf(angle);
    const float s = sinf(angle);
    float *p = x + rh * head_dim + i;
    const float x0 = p[0], x1 = p[1];
    p[0] = x0 * c - x1 * s;
    p[1] = x0 * s + x1 * c;
}

// ---- Q8_0 weights: repack ----------------------------------------------------

// One thread per (row tile, block pair, lane): the lane's 16 quant bytes and,
// for lanes 0..15, the two scales of row (tile*16 + lane) in the pair.
__global__ __launch_bounds__(256) void q8w_repack_kernel(const uint8_t *ggml, int rows, int n_blocks, int n_pairs,
                                                         int64_t n_units, uint8_t *quants, uint16_t *scales) {
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= n_units) return;
    const int lane = (int)(u & 63);
    const int64_t tp = u >> 6;  // tile * n_pairs + pair
    const int pair = (int)(tp % n_pairs);
    const int tile = (int)(tp / n_pairs);
    const int row = tile * 16 + (lane & 15);
    const int kg = lane >> 4;
    uint8_t out[16];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int blk = 2 * pair + j;
        const bool ok = row < rows && blk < n_blocks;
        const uint8_t *src = ggml + ((int64_t)row * n_blocks + blk) * 34 + 2 + kg * 8;
#pragma unroll
        for (int e = 0; e < 8; e++) out[j * 8 + e] = ok ? (uint8_t)(src[e] ^ 0x80) : (uint8_t)0x80;
    }
    uint4 w;
    w.x = out[0] | (out[1] << 8) | (out[2] << 16) | ((uint32_t)out[3] << 24);
    w.y = out[4] | (out[5] << 8) | (out[6] << 16) | ((uint32_t)out[7] << 24);
    w.z = out[8] | (out[9] << 8) | (out[10] << 16) | ((uint32_t)out[11] << 24);
    w.w = out[12] | (out[13] << 8) | (out[14] << 16) | ((uint32_t)out[15] << 24);
    *reinterpret_cast<uint4 *>(quants + u * 16) = w;
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int blk = 2 * pair + j;
            uint16_t sc = 0;
            if (row < rows && blk < n_blocks) {
                const uint8_t *src = ggml + ((int64_t)row * n_blocks + blk) * 34;
                sc = (uint16_t)(src[0] | (src[1] << 8));
            }
            scales[(tp * 16 + lane) * 2 + j] = sc;
        }
    }
}

// ---- activations: f16 pieces ---------------------------------------------------

// Grid (K slices of the split-K kernel, padded vector count / 4), 256
// threads: a workgroup takes 4 consecutive vectors (thread t always vector
// t & 3) and the units (8 elements each) of one K slice, block pairs
// slice*ps .. +ps. Each (vector, slice) takes its own piece scale 2^s from
// the slice's largest |x| alone, so no workgroup waits for another, and the
// split-K kernel undoes it where it already multiplies a slice's sums by
// one factor per vector. Up to kSplitU units per thread stay in registers
// between the maximum and the pieces; a wider slice is read twice. Vectors
// past n_vec get zero pieces. The pieces go out in the B-operand order of
// the MFMA: xp[v / 16][blk][piece][lane = kg*16 + v % 16] = 8 f16 of
// elements blk*32 + kg*8 .. +8 (piece 0 hi, 1 lo), so that one vector
// tile's piece of a block is 1 KiB contiguous and 4 consecutive lanes write
// 4 consecutive 16-byte pieces, one 64-byte request; xs[slice][v] = 2^-s,
// the factor that undoes the scaling.
constexpr int kSplitThreads = 256;
constexpr int kSplitV = 4;                           // vectors per workgroup
constexpr int kSplitStep = kSplitThreads / kSplitV;  // units of a vector per pass
constexpr int kSplitU = 4;                           // units per thread held in registers
template <bool A16>  // x rows 16-byte aligned: float4 loads
__global__ __launch_bounds__(kSplitThreads) void split_x_kernel(const float *x, int n_vec, int cols,
                                                                int n_blocks_pad, int ps, int vec_pad,
                                                                _Float16 *xp, float *xs) {
    const int vq = threadIdx.x & (kSplitV - 1);
    const int v = blockIdx.y * kSplitV + vq;
    const float *xv = x + (int64_t)min(v, n_vec - 1) * cols;
    const int cu = cols / 8;                               // units inside the row (cols is a multiple of 32)
    const int u0 = blockIdx.x * ps * 8;                    // the slice's units: 8 per block pair
    const int u1 = min(n_blocks_pad * 4, u0 + ps * 8);
    const int uin = min(u1, cu);                           // units of the slice inside the row
    const int ut = threadIdx.x / kSplitV;                  // the thread's unit within each pass
    // units past the slice (or the row) are zeros and load nothing: a
    // clamped load there would read other slices' lines again
    auto load_unit = [&](float (&e)[8], int u) {
#pragma unroll
        for (int j = 0; j < 8; j++) e[j] = 0.0f;
        if (v >= n_vec || u >= uin) return;
        const float *src = xv + (int64_t)u * 8;
        if (A16) {
            const float4 a = *reinterpret_cast<const float4 *>(src);
            const float4 b = *reinterpret_cast<const float4 *>(src + 4);
            e[0] = a.x, e[1] = a.y, e[2] = a.z, e[3] = a.w;
            e[4] = b.x, e[5] = b.y, e[6] = b.z, e[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) e[j] = src[j];
        }
    };
    // the largest finite |x|: an infinity keeps its own piece (hi = +-inf,
    // lo = 0) and must not push the finite ones past the f16 range; a NaN
    // stays NaN in its pieces (the reference's block sums give inf / NaN the same way)
    auto finite_max = [](float m, float v) {
        const float a = fabsf(v);
        return a <= 3.402823466e38f ? fmaxf(m, a) : m;
    };
    float e[kSplitU][8];
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < kSplitU; k++) {
        load_unit(e[k], u0 + k * kSplitStep + ut);
#pragma unroll
        for (int j = 0; j < 8; j++) mx = finite_max(mx, e[k][j]);
    }
    for (int u = u0 + kSplitU * kSplitStep + ut; u < uin; u += kSplitStep) {  // the rest of a wide slice
        float t[8];
        load_unit(t, u);
#pragma unroll
        for (int j = 0; j < 8; j++) mx = finite_max(mx, t[j]);
    }
    // maximum over the threads of the same vector: lanes of equal t & 3 in
    // the wave, then the waves
    constexpr int NW = kSplitThreads / 64;
    __shared__ float red[NW][kSplitV];
    for (int o = kSplitV; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((threadIdx.x & 63) < kSplitV) red[threadIdx.x >> 6][vq] = mx;
    __syncthreads();
    mx = red[0][vq];
#pragma unroll
    for (int w = 1; w < NW; w++) mx = fmaxf(mx, red[w][vq]);
    int ex = 0;
    if (mx > 0.0f) frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
    const int sh = 14 - ex;            // the largest finite |x| * 2^sh lies in [2^13, 2^14)
    const float mul = ldexpf(1.0f, sh);
    if (threadIdx.x < kSplitV) xs[(int64_t)blockIdx.x * vec_pad + v] = ldexpf(1.0f, -sh);
    auto put = [&](const float (&t8)[8], int u) {
        half8 hi, lo;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float t = t8[j] * mul;
            const _Float16 h = (_Float16)t;
            hi[j] = h;
            lo[j] = __builtin_isinf(t) ? (_Float16)0.0f : (_Float16)(t - (float)h);
        }
        const int blk = u >> 2;
        const int ln = (u & 3) * 16 + (v & 15);
        _Float16 *dst = xp + (((int64_t)(v >> 4) * n_blocks_pad + blk) * 128 + ln) * 8;
        *reinterpret_cast<half8 *>(dst) = hi;
        *reinterpret_cast<half8 *>(dst + 64 * 8) = lo;
    };
#pragma unroll
    for (int k = 0; k < kSplitU; k++) {
        const int u = u0 + k * kSplitStep + ut;
        if (u < u1) put(e[k], u);
    }
    for (int u = u0 + kSplitU * kSplitStep + ut; u < u1; u += kSplitStep) {
        float t[8];
        load_unit(t, u);
        put(t, u);
    }
}

// ---- the matvec ----------------------------------------------------------------------

// Four consecutive floats as two 8-byte agent-scope loads (bypassing the
// per-XCD L2s, like load_agent; the compiler tracks them in its waits).
__device__ __forceinline__ floatx4 load_agent4(const float *p) {
    uint64_t *q = reinterpret_cast<uint64_t *>(const_cast<float *>(p));
    const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return floatx4{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)), __uint_as_float((uint32_t)b),
                   __uint_as_float((uint32_t)(b >> 32))};
}

// 4 bytes x + 128 -> 4 exact f16 (1024 + byte - 1152) at o[at .. at+3].
__device__ __forceinline__ void bytes_to_h(uint32_t u, half8 &o, int at) {
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x07010700u);  // bytes 0, 1 under 0x64
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x07030702u);  // bytes 2, 3
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const half2v a = __builtin_bit_cast(half2v, lo) - bias;
    const half2v b = __builtin_bit_cast(half2v, hi) - bias;
    o[at] = a[0];
    o[at + 1] = a[1];
    o[at + 2] = b[0];
    o[at + 3] = b[1];
}

constexpr int kMaxVT = 4;        // vector tiles (16 vectors each) per launch
constexpr int kSkWaves = 4;      // waves per workgroup: a quarter of the workgroup's blocks each
constexpr int kSkRT = 4;         // row tiles per wave (and per workgroup): 64 rows share each x fragment
constexpr int kSkMaxSplits = 8;  // K slices per launch (summed by each row group's last workgroup)
constexpr int kSkTargetWgs = 512;

// One K slice of y[v][row] for up to 64 vectors: workgroup (g, s) owns rows
// g*64 .. +64 and the block pairs of slice s, which its four waves split; each
// wave holds 4 row tiles x NVT vector tiles of accumulators, so every x
// fragment it loads serves four row tiles and every weight fragment NVT
// vector tiles. The waves are merged in LDS in a fixed order and the slice's
// sums (times the piece factor of the vector in this slice) go to out[s][vv][row] as agent-scope
// stores, or straight to y when there is one slice; the row group's last
// workgroup to arrive (counted in arrivals[row group]) sums the slices into
// y, so no reduce launch follows. Splitting K across workgroups is what keeps
// the x fragments each CU reads to its slice of x, not all of it.
template <int NVT>
__global__ __launch_bounds__(kSkWaves * 64) void matvec_q8_splitk_kernel(
    const uint8_t *quants, const uint16_t *scales, int rows, int n_tiles, int n_pairs, const _Float16 *xp,
    const float *xs, int xs_stride, int n_blocks_pad, int v0, int n_vec, int n_splits, float *out,
    int64_t split_stride, float *y, int32_t *arrivals) {
    constexpr int RT = kSkRT;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tile0 = blockIdx.x * RT;
    const int kg = lane >> 4;
    const int ps = (n_pairs + n_splits - 1) / n_splits;
    const int q0 = min(n_pairs, (int)blockIdx.y * ps);
    const int q1 = min(n_pairs, q0 + ps);
    const int per = (q1 - q0 + kSkWaves - 1) / kSkWaves;
    const int p0 = min(q1, q0 + wave * per);
    const int p1 = min(q1, p0 + per);

    __shared__ float xsl[NVT * 16];  // this slice's piece factors of the launch's vectors, read by the epilogue
    if ((int)threadIdx.x < NVT * 16) xsl[threadIdx.x] = xs[(int64_t)blockIdx.y * xs_stride + v0 + threadIdx.x];

    floatx4 acc[RT][NVT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int vt = 0; vt < NVT; vt++) acc[rt][vt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // the x pieces of one block for every vector tile: 1 KiB contiguous per piece
    auto load_x = [&](half8 (&bh)[NVT], half8 (&bl)[NVT], int blk) {
#pragma unroll
        for (int vt = 0; vt < NVT; vt++) {
            const _Float16 *src = xp + (((int64_t)(v0 / 16 + vt) * n_blocks_pad + blk) * 128 + lane) * 8;
            bh[vt] = *reinterpret_cast<const half8 *>(src);
            bl[vt] = *reinterpret_cast<const half8 *>(src + 64 * 8);
        }
    };
    // the weights and scales of one block pair for every row tile
    auto load_w = [&](uint4 (&qw)[RT], uint4 (&sw)[RT], int p) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int tile = min(tile0 + rt, n_tiles - 1);
            const int64_t tp = (int64_t)tile * n_pairs + p;
            const u32x4 q = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(quants + (tp * 64 + lane) * 16));
            qw[rt] = make_uint4(q.x, q.y, q.z, q.w);
            sw[rt] = *reinterpret_cast<const uint4 *>(scales + (tp * 16 + kg * 4) * 2);
        }
    };
    // block j of the pair in (qw, sw) against the pieces (bh, bl)
    auto block = [&](const uint4 (&qw)[RT], const uint4 (&sw)[RT], const half8 (&bh)[NVT], const half8 (&bl)[NVT],
                     int j) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const uint4 q = qw[rt];
            const uint4 sv = sw[rt];
            half8 a;
            bytes_to_h(j ? q.z : q.x, a, 0);
            bytes_to_h(j ? q.w : q.y, a, 4);
            // scales of rows kg*4 + r: the lane's 16 bytes hold [row][block] f16
            const uint32_t s01 = j == 0 ? (sv.x & 0xffffu) | (sv.y << 16) : (sv.x >> 16) | (sv.y & 0xffff0000u);
            const uint32_t s23 = j == 0 ? (sv.z & 0xffffu) | (sv.w << 16) : (sv.z >> 16) | (sv.w & 0xffff0000u);
            typedef _Float16 half2v __attribute__((ext_vector_type(2)));
            const half2v h01 = __builtin_bit_cast(half2v, s01);
            const half2v h23 = __builtin_bit_cast(half2v, s23);
            const float sc[4] = {(float)h01[0], (float)h01[1], (float)h23[0], (float)h23[1]};
#pragma unroll
            for (int vt = 0; vt < NVT; vt++) {
                floatx4 c =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh[vt], floatx4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl[vt], c, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[rt][vt][r] = fmaf(c[r], sc[r], acc[rt][vt][r]);
            }
        }
    };

    // software pipeline: the x pieces one block ahead, the weights one pair
    // ahead; every load is unconditional (indices clamped into the wave's
    // range), so none is held back behind a branch
    if (p0 < p1) {
        uint4 qw[RT], sw[RT];
        half8 bh[NVT], bl[NVT];
        load_w(qw, sw, p0);
        load_x(bh, bl, 2 * p0);
        for (int p = p0; p < p1; p++) {
            const int pn = min(p + 1, p1 - 1);
            uint4 qn[RT], sn[RT];
            half8 nh[NVT], nl[NVT];
            load_w(qn, sn, pn);
            load_x(nh, nl, 2 * p + 1);
            block(qw, sw, bh, bl, 0);
            load_x(bh, bl, 2 * pn);
            block(qw, sw, nh, nl, 1);
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                qw[rt] = qn[rt];
                sw[rt] = sn[rt];
            }
        }
    }

    // merge the waves' block ranges in a fixed order
    // (through LDS with padding: 4 floats after every 16 lanes, and tiles of
    // S floats with NVT * S = 16 (mod 64), so that the 64 reads of one wave
    // below, 4 row tiles x 4 lane groups x 4 registers, fall in distinct banks)
    constexpr int S = NVT == 1 ? 272 : (NVT == 2 ? 296 : (NVT == 3 ? 304 : 276));
    static_assert((NVT * S) % 64 == 16 && 4 * 63 + 4 * 3 + 3 < S && S % 4 == 0, "padded tile");
    __shared__ __attribute__((aligned(16))) float red[kSkWaves * RT * NVT * S];
    auto red_at = [&](int w, int rt, int vt, int ln) { return ((w * RT + rt) * NVT + vt) * S + 4 * ln + 4 * (ln >> 4); };
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int vt = 0; vt < NVT; vt++) *reinterpret_cast<floatx4 *>(&red[red_at(wave, rt, vt, lane)]) = acc[rt][vt];
    __syncthreads();
    float *o = out + (int64_t)blockIdx.y * split_stride;
    for (int i = threadIdx.x; i < RT * 16 * NVT * 16; i += kSkWaves * 64) {
        const int rl = i & (RT * 16 - 1);  // row in the workgroup: consecutive threads, consecutive rows
        const int vv = i / (RT * 16);      // vector of the launch
        const int rt = rl >> 4;
        const int rr = rl & 15;
        const int vt = vv >> 4;
        const int ln = (rr >> 2) * 16 + (vv & 15);  // the C lane of (row rr, vector vv & 15)
        const int r = rr & 3;
        float sum = red[red_at(0, rt, vt, ln) + r];
#pragma unroll
        for (int w = 1; w < kSkWaves; w++) sum += red[red_at(w, rt, vt, ln) + r];
        const int row = tile0 * 16 + rl;
        const int v = v0 + vv;
        if (row < rows && v < n_vec) {
            if (arrivals)
                store_agent(o + (int64_t)vv * rows + row, sum * xsl[vv]);
            else
                o[(int64_t)vv * rows + row] = sum * xsl[vv];
        }
    }
    if (!arrivals) return;
    // K slices summed by the last of the row group's workgroups to arrive, in
    // slice order: y = ((s0 + s1) + s2) + ..., the same sums whichever
    // workgroup is last
    __shared__ int lds_last;
    if (!arrive_last(arrivals + blockIdx.x, n_splits, &lds_last)) return;
    constexpr int NQ = RT * 16 * NVT * 16 / 4 / (kSkWaves * 64);  // row quads per thread
    if (rows % 4 == 0 && ((uintptr_t)y & 15) == 0) {  // whole 16-byte row quads
        floatx4 t[NQ][kSkMaxSplits];
#pragma unroll
        for (int k = 0; k < NQ; k++) {
            const int qd = threadIdx.x + k * kSkWaves * 64;
            const int rl = 4 * (qd & (RT * 4 - 1));
            const int vv = qd / (RT * 4);
            const int64_t at = (int64_t)vv * rows + min(tile0 * 16 + rl, rows - 4);
#pragma unroll
            for (int sl = 0; sl < kSkMaxSplits; sl++)
                if (sl < n_splits) t[k][sl] = load_agent4(out + sl * split_stride + at);
        }
#pragma unroll
        for (int k = 0; k < NQ; k++) {
            const int qd = threadIdx.x + k * kSkWaves * 64;
            const int rl = 4 * (qd & (RT * 4 - 1));
            const int vv = qd / (RT * 4);
            const int row = tile0 * 16 + rl;
            floatx4 sum = t[k][0];
#pragma unroll
            for (int sl = 1; sl < kSkMaxSplits; sl++)
                if (sl < n_splits) sum += t[k][sl];
            if (row < rows && v0 + vv < n_vec) *reinterpret_cast<floatx4 *>(y + (int64_t)vv * rows + row) = sum;
        }
    } else {
        for (int i = threadIdx.x; i < RT * 16 * NVT * 16; i += kSkWaves * 64) {
            const int rl = i & (RT * 16 - 1);
            const int vv = i / (RT * 16);
            const int row = tile0 * 16 + rl;
            if (row >= rows || v0 + vv >= n_vec) continue;
            const int64_t at = (int64_t)vv * rows + row;
            float sum = load_agent(out + at);
            for (int sl = 1; sl < n_splits; sl++) sum += load_agent(out + sl * split_stride + at);
            y[at] = sum;
        }
    }
}

template <int NVT>
int launch_splitk(gla_ctx *ctx, const gla_q8w *w, const _Float16 *xp, const float *xs, int xs_stride,
                  int n_blocks_pad, int v0, int n_vec, int n_splits, float *out, int64_t split_stride, float *y,
                  int32_t *arrivals) {
    const dim3 grid((w->n_tiles + kSkRT - 1) / kSkRT, n_splits);
    hipLaunchKernelGGL((matvec_q8_splitk_kernel<NVT>), grid, dim3(kSkWaves * 64), 0, ctx->stream, w->quants,
                       w->scales, w->rows, w->n_tiles, w->n_pairs, xp, xs, xs_stride, n_blocks_pad, v0, n_vec,
                       n_splits, out, split_stride, y, arrivals);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "matvec_q8_splitk_kernel launch: %s", hipGetErrorString(e));
    return GLA_OK;
}

// ---- few vectors: f32 on the vector ALUs -------------------------------------------

constexpr int kFewWaves = 8;        // waves per workgroup: an eighth of the block pairs each
constexpr int kFewBatch = 8;        // block pairs whose weight loads a wave issues together
constexpr int kFewMaxVec = 4;       // vectors per launch
constexpr int kFewLdsFloats = 16384;  // x of the launch's vectors staged in LDS (64 KiB)

// x elements per thread and vector that one staging chunk loads: for
// NV >= 2 one chunk covers the widest row that fits; one vector takes 8 at a
// time. Each vector's LDS row is padded to whole chunks.
__host__ __device__ constexpr int few_xc(int nv) {
    return nv == 1 ? 8 : (kFewLdsFloats / nv + kFewWaves * 64 - 1) / (kFewWaves * 64);
}
__host__ __device__ constexpr int few_stride(int nv, int kpad) {
    return (kpad + few_xc(nv) * kFewWaves * 64 - 1) / (few_xc(nv) * kFewWaves * 64) * (few_xc(nv) * kFewWaves * 64);
}

// y[v][row] for NV (1..4) vectors, one workgroup per 16-row tile: the same
// repacked weights as the MFMA path, with f32 FMAs against x staged once in
// LDS (no activation pieces, no padding to 16 vectors). Lane (row r, group
// kg) covers elements kg*8 .. +8 of both blocks of a pair; each stored byte
// q + 128 becomes the exact f32 q in one signed-byte convert (after one xor
// per four bytes). The two block sums take the row's block scales, then the
// four groups and the waves are summed in a fixed order. Bound: HBM on the
// weights (34 bytes per 32).
template <int NV>
__global__ __launch_bounds__(kFewWaves * 64) void matvec_q8_few_kernel(const uint8_t *quants,
                                                                      const uint16_t *scales, int rows,
                                                                      int n_pairs, int cols, const float *x,
                                                                      float *y) {
    extern __shared__ float xl[];  // [NV][few_stride(NV, n_pairs * 64)], zero past cols
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tile = blockIdx.x;
    const int kg = lane >> 4;
    const int r = lane & 15;
    const int per = (n_pairs + kFewWaves - 1) / kFewWaves;
    const int p0 = min(n_pairs, wave * per);
    const int p1 = min(n_pairs, p0 + per);
    const int kpad = n_pairs * 64;
    const int xstride = few_stride(NV, kpad);

    auto load = [&](uint4 &q, uint32_t &sc, int p) {
        const int64_t tp = (int64_t)tile * n_pairs + p;
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(quants + (tp * 64 + lane) * 16));
        q = make_uint4(v.x, v.y, v.z, v.w);
        sc = *reinterpret_cast<const uint32_t *>(scales + (tp * 16 + r) * 2);  // the row's two block scales
    };
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) acc[v] = 0.0f;
    auto pair = [&](const uint4 &q, uint32_t sc, int p) {
        float w[16];  // q, exact
        const uint32_t qs[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
#pragma unroll
        for (int e = 0; e < 16; e++) w[e] = (float)(int8_t)(qs[e >> 2] >> (8 * (e & 3)));
        typedef _Float16 half2v __attribute__((ext_vector_type(2)));
        const half2v s2 = __builtin_bit_cast(half2v, sc);
        const float s0 = (float)s2[0];
        const float s1 = (float)s2[1];
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const float *xa = xl + v * xstride + p * 64 + kg * 8;  // block 2p
            const float4 a0 = *reinterpret_cast<const float4 *>(xa);
            const float4 a1 = *reinterpret_cast<const float4 *>(xa + 4);
            const float4 b0 = *reinterpret_cast<const float4 *>(xa + 32);  // block 2p + 1
            const float4 b1 = *reinterpret_cast<const float4 *>(xa + 36);
            float t0 = w[0] * a0.x;
            t0 = fmaf(w[1], a0.y, t0);
            t0 = fmaf(w[2], a0.z, t0);
            t0 = fmaf(w[3], a0.w, t0);
            t0 = fmaf(w[4], a1.x, t0);
            t0 = fmaf(w[5], a1.y, t0);
            t0 = fmaf(w[6], a1.z, t0);
            t0 = fmaf(w[7], a1.w, t0);
            float t1 = w[8] * b0.x;
            t1 = fmaf(w[9], b0.y, t1);
            t1 = fmaf(w[10], b0.z, t1);
            t1 = fmaf(w[11], b0.w, t1);
            t1 = fmaf(w[12], b1.x, t1);
            t1 = fmaf(w[13], b1.y, t1);
            t1 = fmaf(w[14], b1.z, t1);
            t1 = fmaf(w[15], b1.w, t1);
            acc[v] = fmaf(t0, s0, acc[v]);
            acc[v] = fmaf(t1, s1, acc[v]);
        }
    };

    // x loads first, all at once into registers, then the first batch of
    // weights: loads return in order, so writing x to LDS waits for x alone
    // while the weights stay in flight
    constexpr int kXC = few_xc(NV);
    constexpr int kChunk = kXC * kFewWaves * 64;  // columns per chunk
    // loads without branches (addresses clamped in bounds, values selected
    // after), so the wait before the LDS writes counts the x loads alone
    float xr[NV][kXC];
#pragma unroll
    for (int v = 0; v < NV; v++)
#pragma unroll
        for (int u = 0; u < kXC; u++) {
            const int c = threadIdx.x + u * kFewWaves * 64;
            const float t = x[(int64_t)v * cols + min(c, cols - 1)];
            xr[v][u] = c < cols ? t : 0.0f;
        }
    uint4 qa[kFewBatch];
    uint32_t sa[kFewBatch];
    const bool whole = p0 + kFewBatch <= p1;
#pragma unroll
    for (int i = 0; i < kFewBatch; i++) load(qa[i], sa[i], min(p0 + i, n_pairs - 1));
#pragma unroll
    for (int v = 0; v < NV; v++)
#pragma unroll
        for (int u = 0; u < kXC; u++) xl[v * xstride + threadIdx.x + u * kFewWaves * 64] = xr[v][u];  // padded row
    for (int c0 = kChunk; NV == 1 && c0 < kpad; c0 += kChunk) {  // rows wider than one chunk
        float xw[NV][kXC];
#pragma unroll
        for (int v = 0; v < NV; v++)
#pragma unroll
            for (int u = 0; u < kXC; u++) {
                const int c = c0 + threadIdx.x + u * kFewWaves * 64;
                const float t = x[(int64_t)v * cols + min(c, cols - 1)];
                xw[v][u] = c < cols ? t : 0.0f;
            }
#pragma unroll
        for (int v = 0; v < NV; v++)
#pragma unroll
            for (int u = 0; u < kXC; u++) xl[v * xstride + c0 + threadIdx.x + u * kFewWaves * 64] = xw[v][u];
    }
    __syncthreads();

    int pb = p0;
    if (whole) {
        for (;;) {
            const int nb = pb + kFewBatch;
            const bool more = nb + kFewBatch <= p1;
            uint4 qb[kFewBatch];
            uint32_t sb[kFewBatch];
            if (more) {
#pragma unroll
                for (int i = 0; i < kFewBatch; i++) load(qb[i], sb[i], nb + i);
            }
#pragma unroll
            for (int i = 0; i < kFewBatch; i++) pair(qa[i], sa[i], pb + i);
            pb = nb;
            if (!more) break;
#pragma unroll
            for (int i = 0; i < kFewBatch; i++) {
                qa[i] = qb[i];
                sa[i] = sb[i];
            }
        }
    }
    for (; pb < p1; pb++) {
        uint4 q;
        uint32_t sc;
        load(q, sc, pb);
        pair(q, sc, pb);
    }

    // the four element groups of each row, then the waves, in a fixed order
#pragma unroll
    for (int v = 0; v < NV; v++) {
        acc[v] += __shfl_xor(acc[v], 16);
        acc[v] += __shfl_xor(acc[v], 32);
    }
    __syncthreads();  // x is no longer read: its LDS holds the waves' sums
    if (lane < 16) {
#pragma unroll
        for (int v = 0; v < NV; v++) xl[(wave * NV + v) * 16 + r] = acc[v];
    }
    __syncthreads();
    if ((int)threadIdx.x < NV * 16) {
        const int v = threadIdx.x >> 4;
        const int rr = threadIdx.x & 15;
        float sum = xl[v * 16 + rr];
#pragma unroll
        for (int w = 1; w < kFewWaves; w++) sum += xl[(w * NV + v) * 16 + rr];
        const int row = tile * 16 + rr;
        if (row < rows) y[(int64_t)v * rows + row] = sum;
    }
}

template <int NV>
int launch_few(gla_ctx *ctx, const gla_q8w *w, const float *x, float *y) {
    const int kpad = w->n_pairs * 64;
    if (NV > 1 && kpad > few_xc(NV) * kFewWaves * 64)  // the kernel stages one chunk per vector when NV > 1
        return set_error(GLA_ERR_KERNEL, "matvec_q8_few_kernel<%d>: %d columns exceed one staging chunk", NV, kpad);
    const size_t lds = (size_t)std::max(NV * few_stride(NV, kpad), kFewWaves * NV * 16) * sizeof(float);
    hipLaunchKernelGGL((matvec_q8_few_kernel<NV>), dim3(w->n_tiles), dim3(kFewWaves * 64), lds, ctx->stream,
                       w->quants, w->scales, w->rows, w->n_pairs, w->cols, x, y);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "matvec_q8_few_kernel launch: %s", hipGetErrorString(e));
    return GLA_OK;
}


int64_t grid_for(int64_t n) { return (n + 255) / 256; }

}  // namespace
}  // namespace gla

using namespace gla;

extern "C" {

int gla_rope(gla_ctx *ctx, float *x, int n_rows, int n_heads, int head_dim, const int32_t *pos, float freq_base,
             float scaling_factor, int rot_dim) {
    if (!ctx || (!x && n_rows > 0) || (!pos && n_rows > 0)) return set_error(GLA_ERR_INVALID, "gla_rope: NULL argument");
    // as the reference: an odd head_dim leaves its last dimension alone, and
    // freq_base / scaling_factor are not checked (0 or negative give inf/NaN there too)
    if (n_rows < 0 || n_heads <= 0 || head_dim <= 0 || rot_dim < 0)
        return set_error(GLA_ERR_INVALID, "gla_rope: bad shape (rows %d, heads %d, head_dim %d, rot_dim %d)", n_rows,
                         n_heads, head_dim, rot_dim);
    const int rot = std::min(rot_dim, head_dim) & ~1;
    const int n_pairs = rot / 2;
    if (n_rows == 0 || n_pairs == 0) return GLA_OK;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    // the context keeps the table of the last (base, head_dim): a model's
    // layers all rotate with the same one
    std::vector<float> &tab = ctx->rope_freq;
    if (memcmp(&ctx->rope_base, &freq_base, sizeof(float)) != 0 || ctx->rope_head_dim != head_dim ||
        (int)tab.size() < n_pairs) {
        tab.resize(n_pairs);
        for (int p = 0; p < n_pairs; p++) tab[p] = 1.0f / powf(freq_base, (float)(2 * p) / (float)head_dim);
        ctx->rope_base = freq_base;
        ctx->rope_head_dim = head_dim;
    }
    for (int p0 = 0; p0 < n_pairs; p0 += kRopeLaunchPairs) {
        const int np = std::min(kRopeLaunchPairs, n_pairs - p0);
        RopeFreqs fr;
        for (int p = 0; p < kRopeLaunchPairs; p++) fr.f[p] = p < np ? tab[p0 + p] : 0.0f;
        const int64_t total = (int64_t)n_rows * n_heads * np;
        hipLaunchKernelGGL(rope_kernel, dim3((unsigned)grid_for(total)), dim3(256), 0, ctx->stream, x, n_rows, n_heads,
                           head_dim, p0, np, pos, scaling_factor, fr);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "rope_kernel launch: %s", hipGetErrorString(e));
    }
    return GLA_OK;
}

int gla_q8w_create(gla_ctx *ctx, const uint8_t *ggml_host, int rows, int cols, gla_q8w **out) {
    if (!ctx || !ggml_host || !out) return set_error(GLA_ERR_INVALID, "gla_q8w_create: NULL argument");
    *out = nullptr;
    if (rows <= 0 || cols <= 0 || cols % 32)
        return set_error(GLA_ERR_INVALID, "gla_q8w_create: rows %d, cols %d (cols must be a positive multiple of 32)",
                         rows, cols);
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    gla_q8w *w = new gla_q8w();
    w->ctx = ctx;
    w->rows = rows;
    w->cols = cols;
    w->n_tiles = (rows + 15) / 16;
    const int n_blocks = cols / 32;
    w->n_pairs = (n_blocks + 1) / 2;
    const int64_t n_units = (int64_t)w->n_tiles * w->n_pairs * 64;
    const size_t raw_bytes = (size_t)rows * n_blocks * 34;
    uint8_t *raw = nullptr;
    hipError_t e = hipMalloc(&w->quants, (size_t)n_units * 16);
    if (e == hipSuccess) e = hipMalloc(&w->scales, (size_t)w->n_tiles * w->n_pairs * 32 * 2);
    if (e == hipSuccess) e = hipMalloc(&raw, raw_bytes);
    if (e == hipSuccess) e = hipMemcpyAsync(raw, ggml_host, raw_bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(q8w_repack_kernel, dim3((unsigned)grid_for(n_units)), dim3(256), 0, ctx->stream, raw, rows,
                           n_blocks, w->n_pairs, n_units, w->quants, w->scales);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (raw) (void)hipFree(raw);
    if (e != hipSuccess) {
        (void)hipFree(w->quants);
        (void)hipFree(w->scales);
        delete w;
        return set_error(GLA_ERR_BUFFER, "gla_q8w_create: %s", hipGetErrorString(e));
    }
    ctx->q8ws.push_back(w);
    *out = w;
    return GLA_OK;
}

int gla_q8w_destroy(gla_q8w *w) {
    if (!w) return GLA_OK;
    if (gla_ctx *ctx = w->ctx) {  // else its context already freed the weights
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        ctx->q8ws.erase(std::remove(ctx->q8ws.begin(), ctx->q8ws.end(), w), ctx->q8ws.end());
        gla::detach_q8w(w);
    }
    delete w;
    return GLA_OK;
}

int gla_matvec_q8_0(gla_ctx *ctx, const gla_q8w *w, const float *x, int n_vec, float *y) {
    if (!ctx || !w || (n_vec > 0 && (!x || !y))) return set_error(GLA_ERR_INVALID, "gla_matvec_q8_0: NULL argument");
    if (w->ctx != ctx)
        return set_error(GLA_ERR_INVALID, "gla_matvec_q8_0: the weights belong to %s",
                         w->ctx ? "another context" : "a destroyed context");
    if (n_vec < 0) return set_error(GLA_ERR_INVALID, "gla_matvec_q8_0: n_vec %d < 0", n_vec);
    if (n_vec == 0) return GLA_OK;
    GLA_CHECK_HIP(hipSetDevice(ctx->device), GLA_ERR_DEVICE);
    const int kpad = w->n_pairs * 64;
    const int few = std::min(kFewMaxVec, kFewLdsFloats / kpad);  // vectors per launch whose x fits in LDS
    if (n_vec <= kFewMaxVec && few >= 1) {
        int rc = GLA_OK;
        for (int v0 = 0; v0 < n_vec && rc == GLA_OK; v0 += few) {
            const float *xv = x + (int64_t)v0 * w->cols;
            float *yv = y + (int64_t)v0 * w->rows;
            switch (std::min(few, n_vec - v0)) {
            case 1:
                rc = launch_few<1>(ctx, w, xv, yv);
                break;
            case 2:
                rc = launch_few<2>(ctx, w, xv, yv);
                break;
            case 3:
                rc = launch_few<3>(ctx, w, xv, yv);
                break;
            default:
                rc = launch_few<4>(ctx, w, xv, yv);
            }
        }
        return rc;
    }
    // split_x_kernel's grid takes 4 vectors per row, at most 65,535 rows
    constexpr int kMaxVec = 65535 * kSplitV / 16 * 16;
    if (n_vec > kMaxVec)
        return set_error(GLA_ERR_INVALID, "gla_matvec_q8_0: n_vec %d > %d (split the call)", n_vec, kMaxVec);
    const int n_blocks_pad = 2 * w->n_pairs;
    const int vec_pad = (n_vec + 15) / 16 * 16;
    const int n_groups = (w->n_tiles + kSkRT - 1) / kSkRT;
    // K slices: enough workgroups to fill the chip, at least one block pair per wave
    const int n_splits = std::max(1, std::min({kSkMaxSplits, (kSkTargetWgs + n_groups / 2) / n_groups,
                                               w->n_pairs / kSkWaves}));
    const size_t xp_bytes = (size_t)vec_pad * n_blocks_pad * 32 * 2 * sizeof(_Float16);  // hi + lo per element
    const int ps = (w->n_pairs + n_splits - 1) / n_splits;  // block pairs per slice, as the split-K kernel takes them
    const size_t xs_bytes = ((size_t)n_splits * vec_pad * sizeof(float) + 255) / 256 * 256;  // [slice][vector]
    const int64_t split_stride = (int64_t)16 * kMaxVT * w->rows;  // one slice of partials: 64 vectors x rows
    const size_t part_bytes = n_splits > 1 ? (size_t)n_splits * split_stride * sizeof(float) : 0;
    void *scr = nullptr;
    int rc = ensure_scratch(ctx, xp_bytes + xs_bytes + part_bytes, &scr);
    if (rc != GLA_OK) return rc;
    _Float16 *xp = (_Float16 *)scr;
    float *xs = (float *)((uint8_t *)scr + xp_bytes);
    float *part = (float *)((uint8_t *)scr + xp_bytes + xs_bytes);
    const dim3 sgrid(n_splits, vec_pad / kSplitV);
    if (((uintptr_t)x & 15) == 0)  // rows start 128-byte apart: the base decides
        hipLaunchKernelGGL(split_x_kernel<true>, sgrid, dim3(kSplitThreads), 0, ctx->stream, x, n_vec, w->cols,
                           n_blocks_pad, ps, vec_pad, xp, xs);
    else
        hipLaunchKernelGGL(split_x_kernel<false>, sgrid, dim3(kSplitThreads), 0, ctx->stream, x, n_vec, w->cols,
                           n_blocks_pad, ps, vec_pad, xp, xs);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GLA_ERR_KERNEL, "split_x_kernel launch: %s", hipGetErrorString(e));
    // K slices summed in the split-K kernel by each row group's last workgroup
    int32_t *arrivals = nullptr;
    if (n_splits > 1) {
        rc = ensure_arrivals(ctx, (size_t)n_groups, &arrivals);
        if (rc != GLA_OK) return rc;
    }
    for (int v0 = 0; v0 < n_vec; v0 += 16 * kMaxVT) {
        const int nvt = std::min(kMaxVT, (n_vec - v0 + 15) / 16);
        float *yv = y + (int64_t)v0 * w->rows;
        float *out = n_splits > 1 ? part : yv;
        switch (nvt) {
        case 1:
            rc = launch_splitk<1>(ctx, w, xp, xs, vec_pad, n_blocks_pad, v0, n_vec, n_splits, out, split_stride, yv,
                                 arrivals);
            break;
        case 2:
            rc = launch_splitk<2>(ctx, w, xp, xs, vec_pad, n_blocks_pad, v0, n_vec, n_splits, out, split_stride, yv,
                                 arrivals);
            break;
        case 3:
            rc = launch_splitk<3>(ctx, w, xp, xs, vec_pad, n_blocks_pad, v0, n_vec, n_splits, out, split_stride, yv,
                                 arrivals);
            break;
        default:
            rc = launch_splitk<4>(ctx, w, xp, xs, vec_pad, n_blocks_pad, v0, n_vec, n_splits, out, split_stride, yv,
                                 arrivals);
        }
        if (rc != GLA_OK) return rc;
    }
    return GLA_OK;
}

int gla_q8w_rows(const gla_q8w *w) { return w ? w->rows : -1; }
int gla_q8w_cols(const gla_q8w *w) { return w ? w->cols : -1; }

}  // extern "C"
