// gla_probe.hip -- achievable-peak probes for the benchmark (not part of the
// attention ABI): a streaming HBM read (one pass over a large buffer, and one
// chunk per launch for the per-launch ceilings of the small workloads) and
// MFMA-only loops, timed with HIP events on the null stream. bench.py reports
// each kernel's throughput both against MI355X's published peaks and against
// these measured ceilings.
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
// clk (when not null): workgroup 0's shader-clock count (s_memtime) and
// 100 MHz real-time count (s_memrealtime) at the start and the end of its loop.
__global__ __launch_bounds__(256) void mfma_bf16_rand_kernel(int iters, float *sink, unsigned long long *clk) {
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
    const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < 8; j++)
            c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j & 3], b[(j + 1) & 3], c[j], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    if (s == 12345.0f) sink[0] = s;
    if (clk && blockIdx.x == 0 && threadIdx.x == 0) {
        const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
        clk[0] = c0;
        clk[1] = c1;
        clk[2] = r0;
        clk[3] = r1;
    }
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

// One read of `chunk` bytes per launch, back to back on the null stream,
// each launch reading the next chunk of `bytes` in rotation (so that with
// bytes past the 256 MB last-level cache every chunk comes from HBM), with
// `wgs` workgroups of the streaming-read kernel; microseconds per launch,
// launch gaps included. chunk and bytes are multiples of 16, chunk <= bytes.
int glp_read_per_launch(const void *buf, size_t bytes, size_t chunk, int wgs, int reps, double *us_out) {
    if (chunk == 0 || chunk % 16 != 0 || chunk > bytes || wgs <= 0 || reps <= 0) return -1;
    uint32_t *sink = nullptr;
    if (hipMalloc(&sink, 4) != hipSuccess) return -3;
    const size_t n_chunks = bytes / chunk;
    size_t next = 0;
    float ms = 0.0f;
    const int rc = time_ms(
        [&] {
            const u32x4 *a = reinterpret_cast<const u32x4 *>(static_cast<const uint8_t *>(buf) + next * chunk);
            next = (next + 1) % n_chunks;
            hipLaunchKernelGGL(stream_read_kernel, dim3(wgs), dim3(256), 0, nullptr, a, chunk / 16, sink);
        },
        reps, &ms);
    (void)hipFree(sink);
    if (rc != 0) return rc;
    *us_out = (double)ms * 1e3;
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
        rc = time_ms([&] { hipLaunchKernelGGL(mfma_bf16_rand_kernel, grid, block, 0, nullptr, iters, sink, nullptr); },
                     3, &ms);
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

// The shader clock the bf16 MFMA loop on random operands runs at (MHz, from
// workgroup 0's s_memtime and s_memrealtime over its loop, one launch after a
// warm-up launch): the matrix units draw more power on random data and the
// part lowers its clock to hold it.
int glp_mfma_clock(int iters, double *mhz_out) {
    unsigned long long *clk = nullptr;
    float *sink = nullptr;
    if (hipMalloc(&clk, 4 * sizeof(unsigned long long)) != hipSuccess) return -3;
    if (hipMalloc(&sink, 4) != hipSuccess) {
        (void)hipFree(clk);
        return -3;
    }
    int n_cu = 0;
    int rc = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || n_cu <= 0) rc = -3;
    unsigned long long h[4] = {0, 0, 0, 0};
    if (rc == 0) {
        for (int i = 0; i < 2; i++)
            hipLaunchKernelGGL(mfma_bf16_rand_kernel, dim3(n_cu * 2), dim3(256), 0, nullptr, iters, sink, clk);
        if (hipDeviceSynchronize() != hipSuccess || hipGetLastError() != hipSuccess ||
            hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess)
            rc = -4;
    }
    (void)hipFree(clk);
    (void)hipFree(sink);
    if (rc != 0) return rc;
    if (h[3] <= h[2]) return -4;
    *mhz_out = (double)(h[1] - h[0]) / ((double)(h[3] - h[2]) / 100.0);
    return 0;
}

}  // extern "C"

