// gla_probe.hip -- achievable-peak probes for the benchmark (not part of the
// attention ABI): a streaming HBM read and MFMA-only loops, timed with HIP
// events on the null stream. bench.py reports each kernel's throughput both
// against MI355X's published peaks and against these measured ceilings.
// A third probe replays the staged bf16 prefill kernel's data movement and
// matrix work over the cfg4 grid with parts switched on and off, to say what
// bounds that kernel (bench.py --prefill-structure).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Grid-stride read of n 16-byte units with non-temporal loads (the decode
// kernels' load kind); the XOR keeps the loads alive.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4 *a, size_t n, uint32_t *sink) {
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * 256 * 4;
    for (size_t i = blockIdx.x * (size_t)1024 + threadIdx.x; i < n; i += stride) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            size_t j = i + (size_t)u * 256;
            j = j < n ? j : i;
            v[u] = __builtin_nontemporal_load(a + j);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

// MFMA-only loops: 8 independent accumulators per wave, `iters` rounds.
__global__ __launch_bounds__(256) void mfma_f32_kernel(int iters, float *sink) {
    floatx4 c[8];
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    const float a = 1.0f + threadIdx.x * 1e-7f, b = 1.0f - threadIdx.x * 1e-7f;
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < 8; j++) c[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c[j], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    if (s == 12345.0f) sink[0] = s;
}

__global__ __launch_bounds__(256) void mfma_bf16_kernel(int iters, float *sink) {
    floatx4 c[8];
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8 a, b;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        a[k] = (__bf16)(1.0f + (threadIdx.x + k) * 1e-3f);
        b[k] = (__bf16)(1.0f - (threadIdx.x + k) * 1e-3f);
    }
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < 8; j++) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c[j], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    if (s == 12345.0f) sink[0] = s;
}

// The bf16 loop on operands of random bits: four (A, B) register pairs per
// lane of roughly N(0, 1) values, a different pair for each accumulator in
// turn. The matrix units draw more power multiplying such data than the
// near-constant operands above, and the part lowers its clock for it, so this
// is the ceiling for attention on real activations.
__global__ __launch_bounds__(256) void mfma_bf16_rand_kernel(int iters, float *sink) {
    floatx4 c[8];
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t st = 0x9e3779b9u ^ (blockIdx.x * 256 + threadIdx.x) * 0x85ebca6bu;
    bf16x8 a[4], b[4];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int k = 0; k < 8; k++) {
            float x[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                // sum of four 8-bit uniforms: mean 0, variance 1 after scaling
                st ^= st << 13;
                st ^= st >> 17;
                st ^= st << 5;
                const float u = (float)(st & 255) + (float)((st >> 8) & 255) + (float)((st >> 16) & 255) +
                                (float)(st >> 24);
                x[h] = (u - 510.0f) * (1.0f / 147.8f);
            }
            a[r][k] = (__bf16)x[0];
            b[r][k] = (__bf16)x[1];
        }
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < 8; j++)
            c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j & 3], b[(j + 1) & 3], c[j], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    if (s == 12345.0f) sink[0] = s;
}

// The fp32 loop on random N(0, 1) operands (as mfma_bf16_rand_kernel).
__global__ __launch_bounds__(256) void mfma_f32_rand_kernel(int iters, float *sink) {
    floatx4 c[8];
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t st = 0x9e3779b9u ^ (blockIdx.x * 256 + threadIdx.x) * 0x85ebca6bu;
    float a[4], b[4];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        st ^= st << 13;
        st ^= st >> 17;
        st ^= st << 5;
        const float u =
            (float)(st & 255) + (float)((st >> 8) & 255) + (float)((st >> 16) & 255) + (float)(st >> 24);
        const float x = (u - 510.0f) * (1.0f / 147.8f);
        if (r < 4)
            a[r] = x;
        else
            b[r - 4] = x;
    }
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < 8; j++) c[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j & 3], b[(j + 1) & 3], c[j], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    if (s == 12345.0f) sink[0] = s;
}

// ---- the staged bf16 prefill's pattern (prefill_bf16s_kernel<128>), cfg4 grid ----
// 32 units x 64 query blocks of 32 (longest first), 4 waves = 4 q-heads, a
// 3-tile LDS ring of 16 KB tile images copied with global_load_lds_dwordx4
// (each wave a quarter), one barrier per tile, S = K.Q^T (16 MFMAs), P as bf16
// (from S, or with a minimal softmax: 2 max + 16 exp2), 2 row-sum MFMAs and
// O += V.P (16 MFMAs). Switches (mode bits): 1 the f32 q rows loaded and
// converted at the start (16 KB per wave), 2 the f32 output rows stored at the
// end (16 KB per wave, whole rows), 4 the minimal softmax, 8 the output stores
// into one 32 KB buffer instead (L2-resident), 16 random inputs (set up by the host). Modes 0-9, 12 and 13,
// each with or without 16. Inputs are synthetic; results
// are discarded. Every access is in bounds: the images are 32 x 64 tiles, q and
// out 32 x 4 x 2048 rows of 128 floats.
constexpr int kPD = 128, kPTile = 128 * kPD, kPRing = 3, kPUnits = 32, kPQ = 2048;

// as the kernel's lds_copy16 (the s_nop: an LDS-DMA load's wait state after an
// SALU write of M0)
__device__ __forceinline__ void p_lds_copy16(const uint8_t *sbase, uint32_t voff, uint32_t m0) {
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
__device__ __forceinline__ void p_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int MODE>
__global__ __launch_bounds__(256, 3) void prefill_pattern_kernel(const uint8_t *img, const float *q, float *out) {
    constexpr int NT = 2, KS = kPD / 32, DT = kPD / 16, CPW = 4;
    __shared__ __attribute__((aligned(16))) uint8_t ring[kPRing][kPTile];
    const int unit = blockIdx.x;
    const int j = (kPQ / 32) - 1 - (int)blockIdx.y;  // query block, longest first
    const int n = j + 1;                              // causal tiles of 32 keys
    const int lane = threadIdx.x & 63, lrow = lane & 15, lgrp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row0 = ((int64_t)unit * 4 + wave) * kPQ + 32 * j;  // the wave's 32 rows
    bf16x8 qb[NT][KS];
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            if (MODE & 1) {
                const float *qp = q + (row0 + nt * 16 + lrow) * kPD + ks * 32 + lgrp * 8;
                const float4 a = *reinterpret_cast<const float4 *>(qp);
                const float4 c = *reinterpret_cast<const float4 *>(qp + 4);
                qb[nt][ks] = bf16x8{(__bf16)a.x, (__bf16)a.y, (__bf16)a.z, (__bf16)a.w,
                                    (__bf16)c.x, (__bf16)c.y, (__bf16)c.z, (__bf16)c.w};
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) qb[nt][ks][e] = (__bf16)(1e-3f * (lane + e + nt + ks));
            }
        }
    floatx4 o[DT][NT], lacc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
#pragma unroll
        for (int t = 0; t < DT; t++) o[t][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        lacc[nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const bf16x8 ones = bf16x8{(__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f,
                               (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f};
    float m = 0.0f;
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)&ring[0][0]);
    const uint8_t *unit_img = img + (int64_t)unit * (kPQ / 32) * kPTile;
    auto issue = [&](int i) {
        const uint8_t *src = unit_img + (int64_t)i * kPTile;
        const uint32_t dst = ring_lds + (uint32_t)((i % kPRing) * kPTile);
#pragma unroll
        for (int c = 0; c < CPW; c++) {
            const int piece = wave * CPW + c;
            p_lds_copy16(src, (uint32_t)(piece * 1024 + lane * 16), dst + piece * 1024);
        }
    };
    for (int i = 0; i < kPRing - 1; i++)
        if (i < n) issue(i);
    for (int i = 0; i < n; i++) {
        if (i + 1 < n)
            p_wait_vm<CPW>();
        else
            p_wait_vm<0>();
        __syncthreads();
        if (i + kPRing - 1 < n) issue(i + kPRing - 1);
        const uint8_t *kimg = ring[i % kPRing];
        const uint8_t *vimg = kimg + 64 * kPD;
        floatx4 sacc[2][NT];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) sacc[mt][nt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            bf16x8 a[2];
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
                a[mt] = *reinterpret_cast<const bf16x8 *>(kimg + ((mt * (kPD / 8) + ks * 4 + lgrp) * 16 + lrow) * 16);
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    sacc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mt], qb[nt][ks], sacc[mt][nt], 0, 0, 0);
        }
        bf16x8 pb[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float pr[2][4];
            if (MODE & 4) {
                m = fmaxf(m, fmaxf(fmaxf(sacc[0][nt][0], sacc[0][nt][1]), fmaxf(sacc[1][nt][2], sacc[1][nt][3])));
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) pr[mt][e] = __builtin_amdgcn_exp2f(sacc[mt][nt][e] - m);
            } else {
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) pr[mt][e] = sacc[mt][nt][e];
            }
            pb[nt] = bf16x8{(__bf16)pr[0][0], (__bf16)pr[0][1], (__bf16)pr[0][2], (__bf16)pr[0][3],
                            (__bf16)pr[1][0], (__bf16)pr[1][1], (__bf16)pr[1][2], (__bf16)pr[1][3]};
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
            lacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[nt], lacc[nt], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < DT; t++) {
            const bf16x8 a = *reinterpret_cast<const bf16x8 *>(vimg + ((t * 4 + lgrp) * 16 + lrow) * 16);
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                o[t][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[nt], o[t][nt], 0, 0, 0);
        }
    }
    const float add = m + lacc[0][0] + lacc[1][0];
    if (MODE & 10) {
        // whole rows through LDS, as the kernel's epilogue
        __syncthreads();
        constexpr int SROW = kPD + 4;
        float *stage = reinterpret_cast<float *>(&ring[0][0]) + wave * 16 * SROW;
        float *dst = (MODE & 8) ? out + (int64_t)(wave * 16) * kPD : out + row0 * kPD;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int t = 0; t < DT; t++)
                *reinterpret_cast<floatx4 *>(stage + lrow * SROW + 16 * t + 4 * lgrp) = o[t][nt] + add;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int r = k * 2 + lane / 32;
                const int c = (lane % 32) * 4;
                const floatx4 v = *reinterpret_cast<const floatx4 *>(stage + r * SROW + c);
                *reinterpret_cast<floatx4 *>(dst + (int64_t)((MODE & 8) ? r : nt * 16 + r) * kPD + c) = v;
            }
        }
    } else if (lane == 0) {
        float s = add;
#pragma unroll
        for (int t = 0; t < DT; t++) s += o[t][0][0] + o[t][1][0];
        if (s == 12345.0f) out[0] = s;
    }
}

template <typename F>
int time_ms(F launch, int reps, float *ms_out) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -2;
    float ms = 0.0f;
    int rc = 0;
    launch();  // warm-up
    if (hipDeviceSynchronize() != hipSuccess || hipEventRecord(e0, nullptr) != hipSuccess) {
        rc = -4;
    } else {
        for (int i = 0; i < reps; i++) launch();
        if (hipEventRecord(e1, nullptr) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
            hipEventElapsedTime(&ms, e0, e1) != hipSuccess || hipGetLastError() != hipSuccess)
            rc = -4;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *ms_out = ms / reps;
    return rc;
}

}  // namespace

extern "C" {

// Read `bytes` (a multiple of 16) from device buffer `buf`; GB/s of one pass.
int glp_stream_read(const void *buf, size_t bytes, int reps, double *gbs_out) {
    uint32_t *sink = nullptr;
    if (hipMalloc(&sink, 4) != hipSuccess) return -3;
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || n_cu <= 0) {
        (void)hipFree(sink);
        return -3;
    }
    const size_t n = bytes / 16;
    float ms = 0.0f;
    const int rc = time_ms(
        [&] {
            hipLaunchKernelGGL(stream_read_kernel, dim3(n_cu * 16), dim3(256), 0, nullptr,
                               static_cast<const u32x4 *>(buf), n, sink);
        },
        reps, &ms);
    (void)hipFree(sink);
    if (rc != 0) return rc;
    *gbs_out = (double)bytes / (ms * 1e-3) / 1e9;
    return 0;
}

// kind 0: v_mfma_f32_16x16x4_f32, kind 1: v_mfma_f32_16x16x32_bf16, kind 2:
// the bf16 loop on random operands, kind 3: the fp32 loop on random operands,
// on 8 waves per CU; TFLOP/s.
int glp_mfma_peak(int kind, int iters, double *tflops_out) {
    float *sink = nullptr;
    if (hipMalloc(&sink, 4) != hipSuccess) return -3;
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || n_cu <= 0) {
        (void)hipFree(sink);
        return -3;
    }
    const dim3 grid(n_cu * 2), block(256);
    float ms = 0.0f;
    int rc;
    double flops_per_mfma;
    if (kind == 0) {
        rc = time_ms([&] { hipLaunchKernelGGL(mfma_f32_kernel, grid, block, 0, nullptr, iters, sink); }, 3, &ms);
        flops_per_mfma = 16.0 * 16 * 4 * 2;
    } else if (kind == 1) {
        rc = time_ms([&] { hipLaunchKernelGGL(mfma_bf16_kernel, grid, block, 0, nullptr, iters, sink); }, 3, &ms);
        flops_per_mfma = 16.0 * 16 * 32 * 2;
    } else if (kind == 2) {
        rc = time_ms([&] { hipLaunchKernelGGL(mfma_bf16_rand_kernel, grid, block, 0, nullptr, iters, sink); }, 3,
                     &ms);
        flops_per_mfma = 16.0 * 16 * 32 * 2;
    } else {
        rc = time_ms([&] { hipLaunchKernelGGL(mfma_f32_rand_kernel, grid, block, 0, nullptr, iters, sink); }, 3,
                     &ms);
        flops_per_mfma = 16.0 * 16 * 4 * 2;
    }
    (void)hipFree(sink);
    if (rc != 0) return rc;
    const double waves = (double)grid.x * 4;
    *tflops_out = waves * iters * 8 * flops_per_mfma / (ms * 1e-3) / 1e12;
    return 0;
}

}  // extern "C"

namespace {
// roughly N(0, 1) from a hashed index: the sum of four 8-bit uniforms
__device__ __forceinline__ float hashed_normal(uint32_t i) {
    uint32_t h = i * 0x9e3779b1u;
    h ^= h >> 15;
    h *= 0x85ebca77u;
    h ^= h >> 13;
    h *= 0xc2b2ae3du;
    h ^= h >> 16;
    const float u = (float)(h & 255) + (float)((h >> 8) & 255) + (float)((h >> 16) & 255) + (float)(h >> 24);
    return (u - 510.0f) * (1.0f / 147.8f);
}

// random pattern inputs: bf16 tile images of N(0, 1) values and f32 q rows of
// N(0, 1) * q_scale (the attention kernel's q carries scale * log2(e))
__global__ __launch_bounds__(256) void fill_random_kernel(__bf16 *img, size_t n_img, float *q, size_t n_q,
                                                           float q_scale) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_img; i += stride)
        img[i] = (__bf16)hashed_normal((uint32_t)i);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_q; i += stride)
        q[i] = q_scale * hashed_normal((uint32_t)i ^ 0x5bd1e995u);
}
}  // namespace

extern "C" {

// The staged bf16 prefill's pattern over the cfg4 grid (prefill_pattern_kernel,
// `mode` bits as above; bit 16: inputs of random N(0, 1) values instead of
// near-constant ones); microseconds per launch, best of `reps` single-launch
// timings after a warm-up.
int glp_prefill_pattern(int mode, int reps, double *us_out) {
    const size_t img_bytes = (size_t)kPUnits * (kPQ / 32) * kPTile;
    const size_t rows_bytes = (size_t)kPUnits * 4 * kPQ * kPD * sizeof(float);
    uint8_t *img = nullptr;
    float *q = nullptr, *out = nullptr;
    int rc = 0;
    if (hipMalloc(&img, img_bytes) != hipSuccess || hipMalloc(&q, rows_bytes) != hipSuccess ||
        hipMalloc(&out, rows_bytes) != hipSuccess) {
        rc = -3;
    } else if (mode & 16) {
        // q * 0.1275 = N(0, 1) rows times d^-1/2 * log2(e) at d = 128
        hipLaunchKernelGGL(fill_random_kernel, dim3(2048), dim3(256), 0, nullptr, reinterpret_cast<__bf16 *>(img),
                           img_bytes / 2, q, rows_bytes / sizeof(float), 0.1275f);
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = -3;
    } else if (hipMemset(img, 0x3c, img_bytes) != hipSuccess || hipMemset(q, 0, rows_bytes) != hipSuccess ||
               hipDeviceSynchronize() != hipSuccess) {
        rc = -3;
    }
    float best = 0.0f;
    for (int r = 0; rc == 0 && r < reps; r++) {
        float ms = 0.0f;
        const dim3 grid(kPUnits, kPQ / 32), block(256);
        auto launch = [&] {
            switch (mode & 15) {
#define GLP_CASE(M) \
    case M: hipLaunchKernelGGL(prefill_pattern_kernel<M>, grid, block, 0, nullptr, img, q, out); break;
                GLP_CASE(0) GLP_CASE(1) GLP_CASE(2) GLP_CASE(3) GLP_CASE(4) GLP_CASE(5) GLP_CASE(6) GLP_CASE(7)
                GLP_CASE(8) GLP_CASE(9) GLP_CASE(12) GLP_CASE(13)
#undef GLP_CASE
            default: break;
            }
        };
        rc = time_ms(launch, 1, &ms);
        if (rc == 0 && (r == 0 || ms < best)) best = ms;
    }
    if (img) (void)hipFree(img);
    if (q) (void)hipFree(q);
    if (out) (void)hipFree(out);
    if (rc != 0) return rc;
    *us_out = best * 1e3;
    return 0;
}

}  // extern "C"
