// Device helpers shared by the kernels of the unity device translation unit.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace svl {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// kernels.rs:380-383 gelu_tanh_value, same constants and evaluation order.
__device__ __forceinline__ float gelu_tanh(float v) {
    float cubic = v * v * v;
    return 0.5f * v * (1.0f + tanhf(0.7978846f * (v + 0.044715f * cubic)));
}

// kernels.rs:767: 1 / sqrt(sum / width + eps).
__device__ __forceinline__ float rms_inverse(float sum_sq, int width, float eps) {
    return 1.0f / sqrtf(sum_sq / (float)width + eps);
}

// audio.rs:1339-1347 clamp_value: the reference's comparisons (NaN passes).
__device__ __forceinline__ float clamp_ref(float v, float lo, float hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

__device__ __forceinline__ f32x4 clamp4(f32x4 v, float lo, float hi) {
    v.x = clamp_ref(v.x, lo, hi);
    v.y = clamp_ref(v.y, lo, hi);
    v.z = clamp_ref(v.z, lo, hi);
    v.w = clamp_ref(v.w, lo, hi);
    return v;
}

// audio.rs:1349-1364 silu_value / sigmoid_value, same branches.
__device__ __forceinline__ float silu_ref(float v) {
    return v >= 0.0f ? v / (1.0f + expf(-v)) : v * expf(v) / (1.0f + expf(v));
}

__device__ __forceinline__ float sigmoid_ref(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

__device__ __forceinline__ void raise_flag(int *flag, int bit) {
    if (flag) atomicOr(flag, bit);
}

__device__ __forceinline__ bool finite4(f32x4 v) {
    return isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w);
}

}  // namespace svl
