// Device helpers shared by the kernels of the unity device translation unit.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace svl {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;

// Values that are the same in every lane (derived from blockIdx and kernel
// arguments) but that the compiler computed in vector registers, moved to
// scalar registers. A buffer resource built from vector registers makes the
// compiler wrap every buffer load in a loop over the distinct values of the
// wave; these keep the resources scalar.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

template <typename T>
__device__ __forceinline__ T *uniform(T *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return (T *)(((uint64_t)hi << 32) | lo);
}


// Reductions over aligned groups of W lanes (W = 4, 16, 32 or 64) on VALU
// lane permutes, with no LDS round trip: DPP within a row of 16 lanes
// (quad_perm xor 1 and xor 2, then the half-row and row mirrors, which pair
// lanes whose quads or halves already agree), v_permlane16_swap and
// v_permlane32_swap across rows (a swap of v with itself leaves
// {v[l], v[l ^ 16]} resp. {v[l], v[l ^ 32]} in its two results). Every lane
// of a group ends with the group's result.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int W, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
    static_assert(W == 4 || W == 16 || W == 32 || W == 64, "group width");
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    v = op(v, dpp_mov<0xB1>(v));   // quad_perm [1, 0, 3, 2]: lane ^ 1
    v = op(v, dpp_mov<0x4E>(v));   // quad_perm [2, 3, 0, 1]: lane ^ 2
    if constexpr (W >= 16) {
        v = op(v, dpp_mov<0x141>(v));  // row_half_mirror: the other quad of the 8
        v = op(v, dpp_mov<0x140>(v));  // row_mirror: the other 8 of the row
    }
    if constexpr (W >= 32) {
        const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
    }
    if constexpr (W == 64) {
        const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
    }
    return v;
}

// Sum / max over the 64 lanes of a wave (every lane active), every lane
// receiving the same bits.
__device__ __forceinline__ float wave_sum(float v) { return group_reduce<64, false>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_reduce<64, true>(v); }

// kernels.rs:380-383 gelu_tanh_value, 0.5 v (1 + tanh u) with the reference's
// constants and u = 0.7978846 (v + 0.044715 v^3), evaluated through the
// identity 0.5 (1 + tanh u) = 1 / (1 + e^(-2u)): v / (1 + e^(-2u)), one
// hardware exponential and one reciprocal. The form has no cancellation at
// either tail (large negative v gives v times a small positive factor, large
// positive v gives v), and its error is a few ulp of the result, against
// the libm tanhf path the reference takes (checked against the oracle at
// 2e-6 over [-6, 6]). Infinite v gives NaN at -inf and +inf at +inf, as the
// reference's formula does.
__device__ __forceinline__ float gelu_tanh(float v) {
    const float cubic = v * v * v;
    const float u = 0.7978846f * (v + 0.044715f * cubic);
    return v * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * u));
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

// audio.rs:1349-1364 silu_value / sigmoid_value. Both branches take the
// exponential of -|v| (exp(-v) for v >= 0, exp(v) otherwise), so it is
// computed once: v >= 0 gives v / (1 + e) and 1 / (1 + e), v < 0 gives
// v * e / (1 + e) and e / (1 + e), the reference's operations on the same
// values (NaN and -0 take the same branch as in the reference).
__device__ __forceinline__ float silu_ref(float v) {
    const float e = expf(-fabsf(v));
    return (v >= 0.0f ? v : v * e) / (1.0f + e);
}

__device__ __forceinline__ float sigmoid_ref(float v) {
    const float e = expf(-fabsf(v));
    return (v >= 0.0f ? 1.0f : e) / (1.0f + e);
}

__device__ __forceinline__ void raise_flag(int *flag, int bit) {
    if (flag) atomicOr(flag, bit);
}

__device__ __forceinline__ bool finite4(f32x4 v) {
    return isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w);
}

// s_waitcnt vmcnt(N): at most N vector-memory operations of this wave in flight.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

}  // namespace svl
