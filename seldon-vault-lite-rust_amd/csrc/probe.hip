// Measured ceilings of the device, for reporting beside the published ones:
//  * FP32 matrix rate: every SIMD of the chip runs independent MFMA
//    accumulator chains from registers (no memory traffic): sixteen
//    v_mfma_f32_16x16x4_f32 chains in one wave per SIMD, and four
//    v_mfma_f32_32x32x2_f32 chains in two waves per SIMD (fewer chains or
//    more waves leave the 16x16x4 pipe partly idle); the faster is reported;
//  * HBM bandwidth: a copy of 1 GiB into another 1 GiB, one float4 per
//    thread over a full grid (bytes read + bytes written per second);
//  * FP64 matrix rate (probe_fp64_peak): eight v_mfma_f64_16x16x4f64 chains
//    in each of four waves per SIMD (one wave per SIMD reaches three
//    quarters of that; more chains per wave change nothing).
// Each is timed with HIP events over several launches after a warm-up; the
// best launch is reported.
#include "svl_internal.hpp"

namespace svl {

template <int CHAINS>
__global__ __launch_bounds__(256) void probe_mfma16_kernel(float *sink, int iters) {
    f32x4 acc[CHAINS];
#pragma unroll
    for (int c = 0; c < CHAINS; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float a = 1e-3f * (float)(threadIdx.x & 63), b = 0.5f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int c = 0; c < CHAINS; ++c)
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CHAINS; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    if (s == -1.f) sink[blockIdx.x] = s;  // never true; keeps the chains live
}

template <int CHAINS>
__global__ __launch_bounds__(256) void probe_mfma32_kernel(float *sink, int iters) {
    f32x16 acc[CHAINS];
#pragma unroll
    for (int c = 0; c < CHAINS; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.f;
    const float a = 1e-3f * (float)(threadIdx.x & 63), b = 0.5f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int c = 0; c < CHAINS; ++c)
            acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CHAINS; ++c) s += acc[c][0] + acc[c][15];
    if (s == -1.f) sink[blockIdx.x] = s;
}

__global__ __launch_bounds__(256) void probe_mfma_f64_kernel(double *sink, int iters) {
    typedef double f64x4 __attribute__((ext_vector_type(4)));
    constexpr int CHAINS = 8;
    f64x4 acc[CHAINS];
#pragma unroll
    for (int c = 0; c < CHAINS; ++c) acc[c] = f64x4{0.0, 0.0, 0.0, 0.0};
    const double a = 1e-3 * (double)(threadIdx.x & 63), b = 0.5;
    // 16 steps per trip: the compiler moves the accumulators between vector
    // and accumulation registers once per trip, which with one step per trip
    // cost more than the MFMAs (the MFMA intrinsic is convergent, so the loop
    // is not unrolled for us)
    for (int i = 0; i < iters; i += 16) {
#pragma unroll
        for (int u = 0; u < 16; ++u)
#pragma unroll
            for (int c = 0; c < CHAINS; ++c)
                acc[c] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc[c], 0, 0, 0);
    }
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < CHAINS; ++c) s += acc[c][0] + acc[c][3];
    if (s == -1.0) sink[blockIdx.x] = s;  // never true; keeps the chains live
}

__global__ __launch_bounds__(256) void probe_copy_kernel(const f32x4 *__restrict__ src,
                                                         f32x4 *__restrict__ dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// Best of `reps` timed launches of `launch` (after one warm-up), in ms.
template <class F>
static hipError_t best_ms(F launch, int reps, hipStream_t s, float *out) {
    hipEvent_t e0, e1;
    hipError_t e = hipEventCreate(&e0);
    if (e != hipSuccess) return e;
    if ((e = hipEventCreate(&e1)) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return e;
    }
    float best = 1e30f;
    launch();
    for (int r = 0; r < reps && e == hipSuccess; ++r) {
        (void)hipEventRecord(e0, s);
        launch();
        (void)hipEventRecord(e1, s);
        if ((e = hipEventSynchronize(e1)) != hipSuccess) break;
        float ms = 0.f;
        if ((e = hipEventElapsedTime(&ms, e0, e1)) == hipSuccess) best = std::min(best, ms);
    }
    if (e == hipSuccess) e = hipGetLastError();
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *out = best;
    return e;
}

hipError_t probe_peaks(double *fp32_mfma_tflops, double *hbm_copy_gbs) {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    hipStream_t s = nullptr;
    if ((e = hipStreamCreate(&s)) != hipSuccess) return e;
    float *sink = nullptr;
    f32x4 *a = nullptr, *b = nullptr;
    const int64_t n4 = (int64_t(1) << 30) / 16;  // 1 GiB of float4
    const int iters = 4000;                       // about 1 ms per launch
    float ms16 = 0.f, ms32 = 0.f, ms = 0.f;
    e = hipMalloc((void **)&sink, (size_t)cus * 2 * sizeof(float));
    if (e == hipSuccess)  // four waves per workgroup: one wave per SIMD
        e = best_ms([&] {
            hipLaunchKernelGGL(probe_mfma16_kernel<16>, dim3(cus), dim3(256), 0, s, sink, iters);
        }, 3, s, &ms16);
    if (e == hipSuccess)  // two waves per SIMD
        e = best_ms([&] {
            hipLaunchKernelGGL(probe_mfma32_kernel<4>, dim3(cus * 2), dim3(256), 0, s, sink,
                               iters / 2);
        }, 3, s, &ms32);
    if (e == hipSuccess) {
        const double f16 = (double)cus * 4 * iters * 16 * (2.0 * 16 * 16 * 4);
        const double f32 = (double)cus * 2 * 4 * (iters / 2) * 4 * (2.0 * 32 * 32 * 2);
        *fp32_mfma_tflops = std::max(f16 / (ms16 * 1e-3), f32 / (ms32 * 1e-3)) / 1e12;
    }
    if (e == hipSuccess) e = hipMalloc((void **)&a, (size_t)n4 * 16);
    if (e == hipSuccess) e = hipMalloc((void **)&b, (size_t)n4 * 16);
    if (e == hipSuccess) e = hipMemsetAsync(a, 0, (size_t)n4 * 16, s);
    if (e == hipSuccess)
        e = best_ms([&] {
            hipLaunchKernelGGL(probe_copy_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                               s, a, b, n4);
        }, 5, s, &ms);
    if (e == hipSuccess) *hbm_copy_gbs = 2.0 * (double)n4 * 16 / (ms * 1e-3) / 1e9;
    (void)hipStreamSynchronize(s);
    (void)hipFree(sink);
    (void)hipFree(a);
    (void)hipFree(b);
    (void)hipStreamDestroy(s);
    return e;
}

hipError_t probe_fp64_peak(double *fp64_mfma_tflops) {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    hipStream_t s = nullptr;
    if ((e = hipStreamCreate(&s)) != hipSuccess) return e;
    double *sink = nullptr;
    const int iters = 12800;  // a multiple of 16; about 12 ms per launch (shorter launches
                              // measured well below the sustained rate)
    float ms = 0.f;
    e = hipMalloc((void **)&sink, (size_t)cus * 4 * sizeof(double));
    if (e == hipSuccess)  // four workgroups of four waves per CU: four waves per SIMD
        e = best_ms([&] {
            hipLaunchKernelGGL(probe_mfma_f64_kernel, dim3(cus * 4), dim3(256), 0, s, sink, iters);
        }, 3, s, &ms);
    if (e == hipSuccess)
        *fp64_mfma_tflops = (double)cus * 4 * 4 * iters * 8 * (2.0 * 16 * 16 * 4) / (ms * 1e-3) / 1e12;
    (void)hipStreamSynchronize(s);
    (void)hipFree(sink);
    (void)hipStreamDestroy(s);
    return e;
}

}  // namespace svl
