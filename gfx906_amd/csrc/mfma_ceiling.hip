// Sustained fp16 MFMA throughput of the GPU this runs on: a measurement aid
// for reading the attention kernel's roofline fraction, not part of the
// attention path (it is built into its own library).
//
// The published MI355X peak (2516.6 TFLOP/s dense fp16) assumes the 2.4 GHz
// shader clock. Under sustained matrix load the card is power-limited and the
// clock it holds depends on the data: operand bits that toggle from one MFMA
// to the next cost energy. This kernel keeps every SIMD's matrix pipe busy
// with independent v_mfma_f32_32x32x16_f16 (two waves per SIMD, one
// workgroup per CU) on
//   mode 0: pseudo-random fp16 operands (|x| < 2.4, eight operand pairs in
//           rotation, so consecutive MFMAs see different data),
//   mode 1: all-zero operands (no toggling: the clock stays near 2.4 GHz),
//   mode 2: mode 0 plus the attention kernel's per-block VALU work (per 16
//           MFMAs: 16 FMA, 16 exp2, 8 fp32->fp16 pack conversions, 8 dot2),
//   mode 3: mode 0's work as v_mfma_f32_16x16x32_f16 (two per 32x32x16, the
//           shape the attention kernel uses),
//   mode 4: mode 3 plus mode 2's VALU work,
// and reports TFLOP/s and the average shader clock over the run (s_memtime
// cycles against the 100 MHz s_memrealtime counter).
#include <hip/hip_runtime.h>

namespace {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 512;     // 8 waves: two per SIMD
constexpr int kLdsHold = 96 * 1024;  // more than half the CU's LDS: one workgroup per CU
constexpr int kMfmaPerIter = 16;

__device__ __forceinline__ unsigned mix32(unsigned x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

// Sum of two 16-bit uniforms, centred: a triangular value in (-2.4, 2.4).
__device__ __forceinline__ f16 operand(unsigned h) {
    const float u = (float)(h & 0xffff) * (1.f / 65536.f) + (float)(h >> 16) * (1.f / 65536.f);
    return (f16)((u - 1.f) * 2.4f);
}

// clk[2*blockIdx.x] = s_memtime cycles, clk[2*blockIdx.x+1] = s_memrealtime
// ticks of wave 0 over the timed loop. sink keeps the results live.
template <int MODE>
__global__ void __launch_bounds__(kThreads, 1)
mfma_ceiling_kernel(unsigned long long* clk, float* sink, int iters) {
    __shared__ char hold[kLdsHold];
    if (iters < 0) hold[threadIdx.x] = 0;  // keeps the allocation; never taken
    const unsigned t = blockIdx.x * kThreads + threadIdx.x;
    f16x8 A[8], B[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            A[i][e] = MODE == 1 ? (f16)0.f : operand(mix32(t * 131u + i * 17u + e));
            B[i][e] = MODE == 1 ? (f16)0.f : operand(mix32(t * 977u + i * 29u + e + 7u));
        }
    f32x16 acc[4] = {};
    f32x4 acc16[8] = {};
    float x[kMfmaPerIter];
#pragma unroll
    for (int i = 0; i < kMfmaPerIter; ++i) x[i] = (float)(mix32(t + i) & 0xff) * (1.f / 256.f) - 4.f;
    float ls = 0.f;
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < kMfmaPerIter; ++j) {
            if (MODE >= 3) {
                acc16[(2 * j) & 7] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    A[j & 7], B[(j + (j >> 3)) & 7], acc16[(2 * j) & 7], 0, 0, 0);
                acc16[(2 * j + 1) & 7] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    A[j & 7], B[(j + (j >> 3) + 3) & 7], acc16[(2 * j + 1) & 7], 0, 0, 0);
            } else {
                acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[j & 7], B[(j + (j >> 3)) & 7],
                                                                    acc[j & 3], 0, 0, 0);
            }
            if (MODE == 2 || MODE == 4) {
                const float p = __builtin_amdgcn_exp2f(fmaf(x[j], 0.127f, -1.f));
                x[j] = p - 0.5f;
                if (j & 1) {
                    const f16x2 h = __builtin_convertvector(f32x2{x[j - 1], p}, f16x2);
                    ls = __builtin_amdgcn_fdot2(h, f16x2{(f16)1.f, (f16)1.f}, ls, false);
                }
            }
        }
    }
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    float s = ls;
#pragma unroll
    for (int i = 0; i < 4; ++i) s += acc[i][0] + acc[i][15];
#pragma unroll
    for (int i = 0; i < 8; ++i) s += acc16[i][0] + acc16[i][3];
    sink[t] = s;
    if (threadIdx.x == 0) {
        clk[2 * blockIdx.x] = c1 - c0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
}

}  // namespace

// Runs `reps` launches of `iters` loop iterations in mode `mode` (0 to 4,
// above) on the current device and stream 0; returns the best launch's
// TFLOP/s (timed with HIP events) and the average shader clock in GHz of the
// last launch. Returns 0 on success, 1 for bad arguments, 2 on a HIP error.
extern "C" int mfma_ceiling(int mode, int iters, int reps, double* tflops, double* ghz) {
    if (mode < 0 || mode > 4 || iters <= 0 || reps <= 0 || !tflops || !ghz) return 1;
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        ncu <= 0)
        return 2;
    unsigned long long* clk = nullptr;
    float* sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 2;
    float best = 1e30f;
    if (hipMalloc(&clk, sizeof(unsigned long long) * 2 * ncu) != hipSuccess) goto done;
    if (hipMalloc(&sink, sizeof(float) * kThreads * ncu) != hipSuccess) goto done;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) goto done;
    for (int r = 0; r < reps; ++r) {
        if (hipEventRecord(e0, 0) != hipSuccess) goto done;
        if (mode == 0)
            hipLaunchKernelGGL(mfma_ceiling_kernel<0>, dim3(ncu), dim3(kThreads), 0, 0, clk, sink, iters);
        else if (mode == 1)
            hipLaunchKernelGGL(mfma_ceiling_kernel<1>, dim3(ncu), dim3(kThreads), 0, 0, clk, sink, iters);
        else if (mode == 2)
            hipLaunchKernelGGL(mfma_ceiling_kernel<2>, dim3(ncu), dim3(kThreads), 0, 0, clk, sink, iters);
        else if (mode == 3)
            hipLaunchKernelGGL(mfma_ceiling_kernel<3>, dim3(ncu), dim3(kThreads), 0, 0, clk, sink, iters);
        else
            hipLaunchKernelGGL(mfma_ceiling_kernel<4>, dim3(ncu), dim3(kThreads), 0, 0, clk, sink, iters);
        if (hipGetLastError() != hipSuccess) goto done;
        if (hipEventRecord(e1, 0) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) goto done;
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) goto done;
        if (ms < best) best = ms;
    }
    {
        unsigned long long* h = new unsigned long long[2 * ncu];
        const bool ok = hipMemcpy(h, clk, sizeof(unsigned long long) * 2 * ncu,
                                  hipMemcpyDeviceToHost) == hipSuccess;
        double cyc = 0, ticks = 0;
        for (int i = 0; ok && i < ncu; ++i) {
            cyc += (double)h[2 * i];
            ticks += (double)h[2 * i + 1];
        }
        delete[] h;
        if (!ok) goto done;
        const double flop = 2.0 * 32 * 32 * 16 * kMfmaPerIter * (double)iters * (kThreads / 64) * ncu;
        *tflops = flop / (best * 1e-3) / 1e12;
        *ghz = ticks > 0 ? cyc / ticks * 0.1 : 0.0;
        rc = 0;
    }
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (clk) (void)hipFree(clk);
    if (sink) (void)hipFree(sink);
    return rc;
}
