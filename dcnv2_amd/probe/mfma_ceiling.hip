// Sustained dense fp16 MFMA rate of the GPU in the issue pattern of the
// warp-specialised forward kernel (512-thread workgroups, one per CU; waves
// 0-3 issue 32 independent 32x32x16 f16 MFMAs per step, one barrier per
// step), for two kinds of operands: all zeros and N(0,1) values.  The MFMA
// pipe draws more power on toggling data and the chip lowers its shader
// clock to stay within its power limit, so the attainable rate depends on the
// data; bench.py reports both rates beside the published peak.  The shader
// clock is read as s_memtime cycles per 100 MHz s_memrealtime tick.
//
// A measurement tool, built into its own library (libdcn2_probe.so); it is not
// part of the operator's C ABI.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <vector>

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMaxGrid = 1024;
__device__ unsigned long long probe_clk[kMaxGrid][4];

__global__ __launch_bounds__(512) void mfma_issue_kernel(const float *__restrict__ in,
                                                         float *__restrict__ out, int steps) {
    const unsigned long long t0 = __builtin_readcyclecounter();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    f16x8 a[2], b[4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[0][e] = (_Float16)in[(lane * 8 + e) & 1023];
        a[1][e] = (_Float16)in[(lane * 8 + e + 512) & 1023];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j][e] = (_Float16)in[1024 + ((lane * 8 + e + j * 256 + blockIdx.x) & 1023)];
    }
    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    if (wave < 4) {
        for (int s = 0; s < steps; ++s) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            __syncthreads();
        }
    } else {
        for (int s = 0; s < steps; ++s) __syncthreads();
    }
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) sum += acc[i][j][r];
    out[blockIdx.x * 512 + threadIdx.x] = sum;
    const unsigned long long t1 = __builtin_readcyclecounter();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        probe_clk[blockIdx.x][0] = t0;
        probe_clk[blockIdx.x][1] = t1;
        probe_clk[blockIdx.x][2] = r0;
        probe_clk[blockIdx.x][3] = r1;
    }
}

}  // namespace

// kind 0: zero operands; 1: N(0,1) operands (fixed seed).  On success stores
// the dense MFMA rate (TFLOP/s, 2*32*32*16 FLOP per MFMA) and the mean shader
// clock (MHz) of the timed launch and returns 0; otherwise returns the HIP
// error code.
extern "C" __attribute__((visibility("default"))) int dcn2_probe_mfma(int kind, int steps,
                                                                     double *tflops, double *mhz) {
    int dev = 0, ncu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    const int grid = ncu < kMaxGrid ? ncu : kMaxGrid;
    std::vector<float> h(2048);
    uint32_t st = 12345u;
    auto uni = [&st]() {
        st = st * 1664525u + 1013904223u;
        return ((st >> 8) + 0.5f) / 16777216.0f;
    };
    for (int i = 0; i < 2048; ++i) {
        const float u1 = uni(), u2 = uni();
        h[i] = kind == 0 ? 0.0f : sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
    }
    float *in = nullptr, *out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    std::vector<unsigned long long> clk((size_t)kMaxGrid * 4);
    if ((e = hipMalloc(&in, h.size() * sizeof(float))) != hipSuccess) return (int)e;
    if ((e = hipMalloc(&out, (size_t)grid * 512 * sizeof(float))) != hipSuccess) goto done;
    if ((e = hipMemcpy(in, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess) goto done;
    if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess) goto done;
    for (int rep = 0; rep < 2; ++rep) {  // the first launch brings the clock to its steady value
        if ((e = hipEventRecord(e0, 0)) != hipSuccess) goto done;
        mfma_issue_kernel<<<grid, 512, 0, 0>>>(in, out, steps);
        if ((e = hipGetLastError()) != hipSuccess) goto done;
        if ((e = hipEventRecord(e1, 0)) != hipSuccess) goto done;
        if ((e = hipEventSynchronize(e1)) != hipSuccess) goto done;
    }
    if ((e = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess) goto done;
    if ((e = hipMemcpyFromSymbol(clk.data(), HIP_SYMBOL(probe_clk), clk.size() * sizeof(unsigned long long), 0,
                                 hipMemcpyDeviceToHost)) != hipSuccess)
        goto done;
    {
        double ratio = 0.0;
        for (int b = 0; b < grid; ++b)
            ratio += (double)(clk[4 * b + 1] - clk[4 * b]) / (double)(clk[4 * b + 3] - clk[4 * b + 2]);
        *mhz = ratio / grid * 100.0;
        *tflops = (double)grid * 4 * steps * 32 * (2.0 * 32 * 32 * 16) / (ms * 1e-3) / 1e12;
    }
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (out) (void)hipFree(out);
    if (in) (void)hipFree(in);
    return (int)e;
}
