// Row kernels of the vision tower (src/model/vision.rs:742-1148). The GEMMs
// (patch projection, fused QKV, O, gate/up + GeGLU, down, text-space
// projection), the residual post-norms and attention reuse the encoder
// kernels; what is specific to the tower lives here:
//  * the patch rescale 2 * (x - 0.5) (vision.rs:767-770);
//  * the two-axis learned position add fused with the first input norm
//    (vision.rs:791-809 and :818-824);
//  * the per-head Q/K RMSNorm + axial RoPE and the unscaled V norm
//    (vision.rs:831-868, 1073-1148);
//  * the 3x3 bin pooling fused with the unscaled norm before the projection
//    (vision.rs:937-944, 980-1040).
// Patches of all images of a batch are packed back to back; every kernel is
// row-local, so images never mix.
#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

// ---- patch rescale ----------------------------------------------------------
__global__ __launch_bounds__(256) void patch_scale_kernel(const float *__restrict__ x,
                                                          float *__restrict__ y, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * 256) {
        const f32x4 v = ((const f32x4 *)x)[i];
        f32x4 r;
        r.x = 2.0f * (v.x - 0.5f);
        r.y = 2.0f * (v.y - 0.5f);
        r.z = 2.0f * (v.z - 0.5f);
        r.w = 2.0f * (v.w - 0.5f);
        ((f32x4 *)y)[i] = r;
    }
}

hipError_t launch_patch_scale(const float *x, float *y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n % 4) return hipErrorInvalidValue;
    const int64_t n4 = n / 4;
    const unsigned grid = (unsigned)std::min<int64_t>((n4 + 255) / 256, 16384);
    hipLaunchKernelGGL(patch_scale_kernel, dim3(grid), dim3(256), 0, s, x, y, n4);
    return hipGetLastError();
}

// ---- position add + first input norm ----------------------------------------
// h[t] += table[0][x_t] + table[1][y_t]   (the two table rows summed first,
// as vision.rs:806-808 does), then n[t] = rms(h[t], w). One wave per patch.
template <int NC>
__global__ __launch_bounds__(256) void patch_pos_kernel(float *__restrict__ h,
                                                        const int32_t *__restrict__ pos,
                                                        const float *__restrict__ table,
                                                        int64_t pos_size,
                                                        const float *__restrict__ w,
                                                        float *__restrict__ n, int64_t rows,
                                                        int width, float eps, int *flag) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nv = width >> 2;
    const int px = pos[2 * row], py = pos[2 * row + 1];
    const f32x4 *tx = (const f32x4 *)(table + (int64_t)px * width);
    const f32x4 *ty = (const f32x4 *)(table + (pos_size + py) * (int64_t)width);
    f32x4 *hr = (f32x4 *)(h + row * width);
    f32x4 v[NC];
    float ss = 0.f;
    bool ok = true;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            v[c] = hr[i] + (tx[i] + ty[i]);
            hr[i] = v[c];
            ok = ok && finite4(v[c]);
            ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
        }
    }
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, width, eps);
    ok = ok && isfinite(ss);
    f32x4 *nr = (f32x4 *)(n + row * width);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            const f32x4 y = v[c] * inv * ((const f32x4 *)w)[i];
            ok = ok && finite4(y);
            nr[i] = y;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_patch_pos(float *h, const int32_t *pos, const float *table, int64_t pos_size,
                            const float *w, float *n, int64_t rows, int width, float eps,
                            int *flag, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (width % 4 || width > 2048) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4));
    switch ((width + 255) / 256) {
        case 1: hipLaunchKernelGGL(patch_pos_kernel<1>, grid, dim3(256), 0, s, h, pos, table, pos_size, w, n, rows, width, eps, flag); break;
        case 2: hipLaunchKernelGGL(patch_pos_kernel<2>, grid, dim3(256), 0, s, h, pos, table, pos_size, w, n, rows, width, eps, flag); break;
        case 3: hipLaunchKernelGGL(patch_pos_kernel<3>, grid, dim3(256), 0, s, h, pos, table, pos_size, w, n, rows, width, eps, flag); break;
        case 4: hipLaunchKernelGGL(patch_pos_kernel<4>, grid, dim3(256), 0, s, h, pos, table, pos_size, w, n, rows, width, eps, flag); break;
        default: hipLaunchKernelGGL(patch_pos_kernel<8>, grid, dim3(256), 0, s, h, pos, table, pos_size, w, n, rows, width, eps, flag); break;
    }
    return hipGetLastError();
}

// ---- per-head norm + axial RoPE ------------------------------------------
// One wave per (patch, head slot) of the fused [q | k | v] row. Slots
// [0, nh) are query heads (RMSNorm with qn, then axial RoPE), [nh, nh + nkv)
// key heads (kn, RoPE), the rest value heads (unscaled RMSNorm). Each lane
// owns whole rotation pairs (e0, e0 + hd/4) of one half, so the in-place
// update needs no exchange: the row's sum of squares is reduced before any
// lane writes. Half 0 rotates by the patch's x, half 1 by its y, with the
// angle tables cos_t / sin_t [coordinate, hd/4] built on the host.
__global__ __launch_bounds__(256) void qkv_post_axial_kernel(
    float *__restrict__ qkv, int64_t ld, int64_t tokens, int nh, int nkv, int hd,
    const float *__restrict__ qn, const float *__restrict__ kn, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int32_t *__restrict__ pos, float eps, int *flag) {
    const int slots = nh + 2 * nkv;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= tokens * slots) return;
    const int64_t t = r / slots;
    const int slot = (int)(r - t * slots);
    float *row = qkv + t * ld + (int64_t)slot * hd;
    const float *w = slot < nh ? qn : (slot < nh + nkv ? kn : nullptr);
    float ss = 0.f;
    for (int i = lane; i < hd; i += 64) ss += row[i] * row[i];
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, hd, eps);
    bool ok = isfinite(ss);
    const int half = hd / 2, quarter = hd / 4;
    if (w) {
        const int px = pos[2 * t], py = pos[2 * t + 1];
        for (int j = lane; j < half; j += 64) {
            const int hf = j >= quarter, i = j - hf * quarter;
            const int e0 = hf * half + i, e1 = e0 + quarter;
            const int64_t ti = (int64_t)(hf ? py : px) * quarter + i;
            const float c = cos_t[ti], sn = sin_t[ti];
            const float f = row[e0] * inv * w[e0];
            const float g = row[e1] * inv * w[e1];
            const float y0 = f * c - g * sn;
            const float y1 = g * c + f * sn;
            ok = ok && isfinite(y0) && isfinite(y1);
            row[e0] = y0;
            row[e1] = y1;
        }
    } else {
        for (int i = lane; i < hd; i += 64) {
            const float y = row[i] * inv;
            ok = ok && isfinite(y);
            row[i] = y;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

// The same per (token, slot) row for head_dim 16 * EPL (64, 128, 256), four
// rows per wave: lane s of a row's 16 holds elements s, s + 16, ..., so each
// rotation pair (e, e + hd / 4) sits in one lane and the sum of squares
// reduces over 16 lanes. At head_dim 64 one row per wave left 3/4 of the
// wave idle through its reduction and dependent loads.
template <int EPL>
__global__ __launch_bounds__(256) void qkv_post_axial_rows_kernel(
    float *__restrict__ qkv, int64_t ld, int64_t tokens, int nh, int nkv,
    const float *__restrict__ qn, const float *__restrict__ kn, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int32_t *__restrict__ pos, float eps, int *flag) {
    constexpr int RL = 16, HD = RL * EPL, HALF = HD / 2, QUARTER = HD / 4;
    static_assert(QUARTER % RL == 0, "rotation pairs share a lane");
    const int slots = nh + 2 * nkv;
    const int lane = threadIdx.x & 63, sub = lane & (RL - 1);
    const int64_t r = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
    if (r >= tokens * slots) return;  // whole 16-lane groups: the reductions stay within a group
    const int64_t t = r / slots;
    const int slot = (int)(r - t * slots);
    float *row = qkv + t * ld + (int64_t)slot * HD;
    const float *w = slot < nh ? qn : (slot < nh + nkv ? kn : nullptr);
    float v[EPL];
    float ss = 0.f;
#pragma unroll
    for (int m = 0; m < EPL; ++m) {
        v[m] = row[sub + RL * m];
        ss += v[m] * v[m];
    }
#pragma unroll
    for (int o = RL / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, RL);
    const float inv = rms_inverse(ss, HD, eps);
    bool ok = isfinite(ss);
    if (w) {
        const int px = pos[2 * t], py = pos[2 * t + 1];
#pragma unroll
        for (int m0 = 0; m0 < EPL; ++m0) {
            if ((RL * m0) % HALF >= QUARTER) continue;  // m0 holds the pair's first element
            constexpr int DM = QUARTER / RL;
            const int m1 = m0 + DM;
            const int e0 = sub + RL * m0, e1 = e0 + QUARTER;
            const int hf = e0 >= HALF, i = e0 - hf * HALF;
            const int64_t ti = (int64_t)(hf ? py : px) * QUARTER + i;
            const float c = cos_t[ti], sn = sin_t[ti];
            const float f = v[m0] * inv * w[e0];
            const float g = v[m1] * inv * w[e1];
            const float y0 = f * c - g * sn;
            const float y1 = g * c + f * sn;
            ok = ok && isfinite(y0) && isfinite(y1);
            row[e0] = y0;
            row[e1] = y1;
        }
    } else {
#pragma unroll
        for (int m = 0; m < EPL; ++m) {
            const float y = v[m] * inv;
            ok = ok && isfinite(y);
            row[sub + RL * m] = y;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_qkv_post_axial(float *qkv, int64_t ld, int64_t tokens, int nh, int nkv, int hd,
                                 const float *qn, const float *kn, const float *cos_t,
                                 const float *sin_t, const int32_t *pos, float eps, int *flag,
                                 hipStream_t s) {
    if (tokens <= 0) return hipSuccess;
    if (hd % 4) return hipErrorInvalidValue;
    const int64_t rows = tokens * (nh + 2 * nkv);
    const dim3 grid16((unsigned)((rows + 15) / 16));
#define QPA_LAUNCH(EPL)                                                                       \
    hipLaunchKernelGGL(qkv_post_axial_rows_kernel<EPL>, grid16, dim3(256), 0, s, qkv, ld, tokens, \
                       nh, nkv, qn, kn, cos_t, sin_t, pos, eps, flag)
    switch (hd) {
        case 64: QPA_LAUNCH(4); break;
        case 128: QPA_LAUNCH(8); break;
        case 256: QPA_LAUNCH(16); break;
        default:
            hipLaunchKernelGGL(qkv_post_axial_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                               s, qkv, ld, tokens, nh, nkv, hd, qn, kn, cos_t, sin_t, pos, eps, flag);
    }
#undef QPA_LAUNCH
    return hipGetLastError();
}

// ---- 3x3 bin pooling + unscaled norm ----------------------------------------
// One workgroup per soft token s: the patches of its bin (bin_patch
// [bin_start[s], bin_start[s+1]), in patch order) are summed per column in
// that order from 0, as vision.rs:1019-1026 accumulates them; then
// v = (sum / 9) * scale (vision.rs:1034-1036) and out = v * rms_inverse(v)
// (rms_norm_rows_unscaled). Columns c = tid + 256 k, width <= 2048.
__global__ __launch_bounds__(256) void pool_bins_kernel(const float *__restrict__ h,
                                                        const int32_t *__restrict__ bin_start,
                                                        const int32_t *__restrict__ bin_patch,
                                                        int width, float divisor, float scale,
                                                        float eps, float *__restrict__ out,
                                                        int *flag) {
    __shared__ float red[4];
    const int s = blockIdx.x, tid = threadIdx.x;
    const int k0 = bin_start[s], k1 = bin_start[s + 1];
    float v[8];
    float ss = 0.f;
    bool ok = true;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int col = tid + 256 * c;
        v[c] = 0.f;
        if (col < width) {
            float acc = 0.0f;
            for (int k = k0; k < k1; ++k) acc += h[(int64_t)bin_patch[k] * width + col];
            v[c] = (acc / divisor) * scale;
            ok = ok && isfinite(v[c]);
            ss += v[c] * v[c];
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = rms_inverse(ss, width, eps);
    ok = ok && isfinite(ss);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int col = tid + 256 * c;
        if (col < width) {
            const float y = v[c] * inv;
            ok = ok && isfinite(y);
            out[(int64_t)s * width + col] = y;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_pool_bins(const float *h, const int32_t *bin_start, const int32_t *bin_patch,
                            int64_t soft_tokens, int width, float divisor, float scale, float eps,
                            float *out, int *flag, hipStream_t s) {
    if (soft_tokens <= 0) return hipSuccess;
    if (width > 2048) return hipErrorInvalidValue;
    hipLaunchKernelGGL(pool_bins_kernel, dim3((unsigned)soft_tokens), dim3(256), 0, s, h,
                       bin_start, bin_patch, width, divisor, scale, eps, out, flag);
    return hipGetLastError();
}

}  // namespace svl
