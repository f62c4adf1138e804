// Row kernels of the audio tower (src/model/audio.rs:981-1690). The
// projections are the shared GEMM with the clipped-linear epilogues; what is
// specific to the tower lives here:
//  * the two stride-2 3x3 subsampling convolutions, each with its per-position
//    LayerNorm (weight, no bias) and ReLU (audio.rs:1136-1255, 1290-1322):
//    the first direct, the second as im2col + the MFMA GEMM;
//  * one fused row kernel for every clamp / RMSNorm / residual / next-norm
//    chain of the conformer block (audio.rs:1374-1433, 1000-1066);
//  * the chunked local attention with relative positions and the logit soft
//    cap (audio.rs:1529-1669);
//  * the light convolution's causal depthwise conv + clamp + RMSNorm + SiLU
//    (audio.rs:1448-1527);
//  * the output tail's unscaled RMSNorm over valid tokens (audio.rs:1085-1133).
// Clips are packed back to back; every kernel stays within a clip.
#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

constexpr int MEL_BINS = 128;
constexpr int FREQ0 = 64;  // after the first stride-2 convolution
constexpr int FREQ1 = 32;  // after the second

// ---- subsampling convolution 0: 1 -> C0 channels + LayerNorm + ReLU -------
// One wave per (layer-0 row, frequency); lane l holds channels l, l+64, ...
template <int NCH>
__global__ __launch_bounds__(256) void sscp_conv0_kernel(const float *__restrict__ mel,
                                                         const uint8_t *__restrict__ mask,
                                                         const SscpRow *__restrict__ rows,
                                                         int64_t n_rows, const float *__restrict__ w,
                                                         const float *__restrict__ ln, int C0,
                                                         float eps, float *__restrict__ out,
                                                         int *flag) {
    const int64_t pos = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (pos >= n_rows * FREQ0) return;
    const int64_t r = pos / FREQ0;
    const int f = (int)(pos - r * FREQ0);
    const SscpRow ri = rows[r];
    float tap[9];
#pragma unroll
    for (int kt = 0; kt < 3; ++kt)
#pragma unroll
        for (int kf = 0; kf < 3; ++kf) {
            const int it = 2 * ri.t + kt - 1, iff = 2 * f + kf - 1;
            const bool ok = it >= 0 && it < ri.len && iff >= 0 && iff < MEL_BINS &&
                            mask[ri.base + it];
            tap[kt * 3 + kf] = ok ? mel[(int64_t)(ri.base + it) * MEL_BINS + iff] : 0.0f;
        }
    float v[NCH];
    float s = 0.f;
    bool ok = true;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        const int c = lane + 64 * j;
        v[j] = 0.f;
        if (c < C0) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 9; ++k) acc += tap[k] * w[c * 9 + k];
            v[j] = acc;
            ok = ok && isfinite(acc);
            s += acc;
        }
    }
    const float mean = wave_sum(s) / (float)C0;
    float var = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        const int c = lane + 64 * j;
        if (c < C0) {
            const float d = v[j] - mean;
            var += d * d;
        }
    }
    var = wave_sum(var) / (float)C0;
    const float inv = 1.0f / sqrtf(var + eps);
    ok = ok && isfinite(inv);
    float *o = out + pos * C0;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        const int c = lane + 64 * j;
        if (c < C0) o[c] = fmaxf((v[j] - mean) * inv * ln[c], 0.0f);
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_sscp_conv0(const float *mel, const uint8_t *mask, const SscpRow *rows,
                             int64_t n_rows, const float *w, const float *ln, int C0, float eps,
                             float *out, int *flag, hipStream_t s) {
    if (n_rows <= 0) return hipSuccess;
    const dim3 grid((unsigned)((n_rows * FREQ0 + 3) / 4));
    switch ((C0 + 63) / 64) {
        case 1: hipLaunchKernelGGL(sscp_conv0_kernel<1>, grid, dim3(256), 0, s, mel, mask, rows, n_rows, w, ln, C0, eps, out, flag); break;
        case 2: hipLaunchKernelGGL(sscp_conv0_kernel<2>, grid, dim3(256), 0, s, mel, mask, rows, n_rows, w, ln, C0, eps, out, flag); break;
        case 3: case 4: hipLaunchKernelGGL(sscp_conv0_kernel<4>, grid, dim3(256), 0, s, mel, mask, rows, n_rows, w, ln, C0, eps, out, flag); break;
        case 5: case 6: case 7: case 8: hipLaunchKernelGGL(sscp_conv0_kernel<8>, grid, dim3(256), 0, s, mel, mask, rows, n_rows, w, ln, C0, eps, out, flag); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- subsampling convolution 1 as im2col + GEMM ---------------------------
// col[(r * 32 + f) * 9 C0 + ic * 9 + kt * 3 + kf] = layer0 input tap, zero
// where the tap is outside the clip, masked or outside the 64 frequencies:
// the k order of the layer-1 weight [C1][C0][3][3], so the GEMM against it
// sums each output in the reference's (channel, row, column) order. One
// thread per (output position, input channel): coalesced reads over ic.
__global__ __launch_bounds__(256) void sscp_im2col_kernel(const float *__restrict__ l0,
                                                          const uint8_t *__restrict__ mask0,
                                                          const SscpRow *__restrict__ rows,
                                                          int64_t n_rows, int C0,
                                                          float *__restrict__ col) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n_rows * FREQ1 * C0) return;
    const int ic = (int)(idx % C0);
    const int64_t pos = idx / C0;
    const int64_t r = pos / FREQ1;
    const int f = (int)(pos - r * FREQ1);
    const SscpRow ri = rows[r];
    float *dst = col + pos * (int64_t)(9 * C0) + ic * 9;
#pragma unroll
    for (int kt = 0; kt < 3; ++kt) {
        const int it = 2 * ri.t + kt - 1;
        const bool row_ok = it >= 0 && it < ri.len && mask0[ri.base + it];
#pragma unroll
        for (int kf = 0; kf < 3; ++kf) {
            const int iff = 2 * f + kf - 1;
            const bool ok = row_ok && iff >= 0 && iff < FREQ0;
            dst[kt * 3 + kf] = ok ? l0[((int64_t)(ri.base + it) * FREQ0 + iff) * C0 + ic] : 0.0f;
        }
    }
}

hipError_t launch_sscp_im2col(const float *l0, const uint8_t *mask0, const SscpRow *rows,
                              int64_t n_rows, int C0, float *col, hipStream_t s) {
    const int64_t n = n_rows * FREQ1 * C0;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(sscp_im2col_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, l0,
                       mask0, rows, n_rows, C0, col);
    return hipGetLastError();
}

// LayerNorm (weight, no bias) + ReLU over the C channels of each of `n`
// positions, in place; one wave per position.
__global__ __launch_bounds__(256) void sscp_ln_relu_kernel(float *__restrict__ x,
                                                           const float *__restrict__ ln, int C,
                                                           int64_t n, float eps, int *flag) {
    const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (p >= n) return;
    float *row = x + p * C;
    float s = 0.f;
    bool ok = true;
    for (int c = lane; c < C; c += 64) {
        ok = ok && isfinite(row[c]);
        s += row[c];
    }
    const float mean = wave_sum(s) / (float)C;
    float var = 0.f;
    for (int c = lane; c < C; c += 64) {
        const float d = row[c] - mean;
        var += d * d;
    }
    var = wave_sum(var) / (float)C;
    const float inv = 1.0f / sqrtf(var + eps);
    ok = ok && isfinite(inv);
    for (int c = lane; c < C; c += 64) row[c] = fmaxf((row[c] - mean) * inv * ln[c], 0.0f);
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_sscp_ln_relu(float *x, const float *ln, int C, int64_t n, float eps, int *flag,
                               hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(sscp_ln_relu_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, x, ln,
                       C, n, eps, flag);
    return hipGetLastError();
}

// ---- fused clamp / RMSNorm / residual chain ---------------------------------
//   t = w1 ? rms(clamp(x, +-c1), w1) : x
//   h = res ? res + t * rw : t            (stored when h_out)
//   n = rms(clamp(h, +-c2), w2)           (stored when w2)
// res, h_out and n_out may alias each other (each lane reads its own elements
// before writing them). One wave per row, width % 4 == 0, width <= 2048.
template <int NC>
__global__ __launch_bounds__(256) void audio_rows_kernel(
    const float *x, float c1, const float *__restrict__ w1, const float *res, float rw,
    float *h_out, float c2, const float *__restrict__ w2, float *n_out, int64_t rows, int width,
    float eps, int *flag) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nv = width >> 2;
    const f32x4 *xr = (const f32x4 *)(x + row * width);
    f32x4 v[NC];
    bool ok = true;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            v[c] = xr[i];
            if (w1) {
                v[c] = clamp4(v[c], -c1, c1);
                ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
            }
        }
    }
    if (w1) {
        ss = wave_sum(ss);
        const float inv = rms_inverse(ss, width, eps);
        ok = ok && isfinite(ss);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int i = lane + 64 * c;
            if (i < nv) v[c] = v[c] * inv * ((const f32x4 *)w1)[i];
        }
    }
    float ss2 = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            if (res) v[c] = ((const f32x4 *)(res + row * width))[i] + v[c] * rw;
            ok = ok && finite4(v[c]);
            if (h_out) ((f32x4 *)(h_out + row * width))[i] = v[c];
            if (w2) {
                const f32x4 y = clamp4(v[c], -c2, c2);
                v[c] = y;
                ss2 += y.x * y.x + y.y * y.y + y.z * y.z + y.w * y.w;
            }
        }
    }
    if (w2) {
        ss2 = wave_sum(ss2);
        const float inv = rms_inverse(ss2, width, eps);
        ok = ok && isfinite(ss2);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int i = lane + 64 * c;
            if (i < nv) {
                const f32x4 y = v[c] * inv * ((const f32x4 *)w2)[i];
                ok = ok && finite4(y);
                ((f32x4 *)(n_out + row * width))[i] = y;
            }
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_audio_rows(const float *x, float c1, const float *w1, const float *res, float rw,
                             float *h_out, float c2, const float *w2, float *n_out, int64_t rows,
                             int width, float eps, int *flag, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (width % 4 || width > 2048) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4));
#define AR_LAUNCH(NC)                                                                          \
    hipLaunchKernelGGL(audio_rows_kernel<NC>, grid, dim3(256), 0, s, x, c1, w1, res, rw, h_out, \
                       c2, w2, n_out, rows, width, eps, flag)
    switch ((width + 255) / 256) {
        case 1: AR_LAUNCH(1); break;
        case 2: AR_LAUNCH(2); break;
        case 3: AR_LAUNCH(3); break;
        case 4: AR_LAUNCH(4); break;
        case 5: case 6: AR_LAUNCH(6); break;
        default: AR_LAUNCH(8); break;
    }
#undef AR_LAUNCH
    return hipGetLastError();
}

// ---- chunked local attention ---------------------------------------------
// One wave per (row, head). Lane l holds head dims l, l+64, ... of the
// scaled query (q * qf[d], qf = q_scale * softplus(per_dim_scale)) and keys
// are scaled by k_scale as they are read. Context entry ci of the row's block
// is key block*chunk + ci - (left-1) of the same clip; it is valid when that
// key is in the clip, unmasked, and 0 <= query - key < left - 1. The score
// is tanh((q.k + q.relk[ci - offset]) / cap) * cap; lane ci keeps score ci
// (context <= 64). Masked query rows get zeros.
__global__ __launch_bounds__(256) void audio_attn_kernel(AudioAttnArgs p) {
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (wid >= p.rows * p.heads) return;
    const int64_t i = wid / p.heads;
    const int h = (int)(wid - i * p.heads);
    const int hd = p.head_dim;
    float *orow = p.out + i * p.ldo + (int64_t)h * hd;
    if (!p.mask[i]) {
        for (int d = lane; d < hd; d += 64) orow[d] = 0.0f;
        return;
    }
    const int il = p.pos[i], len = p.rowlen[i];
    const int64_t base = i - il;
    const int block = il / p.chunk, off = il - block * p.chunk;
    const int max_past = p.left - 1, left_window = p.left - 1;
    const float *qrow = p.q + i * p.ldq + (int64_t)h * hd;
    float q[4];  // hd <= 256
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        q[j] = d < hd ? qrow[d] * p.qf[d] : 0.0f;
    }
    float my = -INFINITY;
    for (int ci = 0; ci < p.context; ++ci) {
        const int kl = block * p.chunk + ci - max_past;
        const bool valid = kl >= 0 && kl < len && p.mask[base + kl] && il - kl >= 0 &&
                           il - kl < left_window;
        float score = -1.0e9f;
        if (valid) {
            const float *krow = p.k + (base + kl) * p.ldk + (int64_t)h * hd;
            const int rel = ci - off;
            const bool has_rel = rel >= 0 && rel < p.positions;
            const float *rrow = p.relk + ((int64_t)(has_rel ? rel : 0) * p.heads + h) * hd;
            float part = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = lane + 64 * j;
                if (d < hd) {
                    part += q[j] * (krow[d] * p.k_scale);
                    if (has_rel) part += q[j] * rrow[d];
                }
            }
            const float dot = wave_sum(part);
            score = tanhf(dot / p.cap) * p.cap;
        }
        if (lane == ci) my = score;
    }
    const float maximum = wave_max(lane < p.context ? my : -INFINITY);
    if (maximum <= -1.0e9f / 2.0f) {
        for (int d = lane; d < hd; d += 64) orow[d] = 0.0f;
        return;
    }
    const float e = lane < p.context ? expf(my - maximum) : 0.0f;
    const float sum = wave_sum(e);
    bool ok = isfinite(sum) && sum > 0.0f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int ci = 0; ci < p.context; ++ci) {
        const float wgt = __shfl(e, ci, 64) / sum;
        const int kl = block * p.chunk + ci - max_past;
        if (wgt == 0.0f || kl < 0 || kl >= len) continue;
        const float *vrow = p.v + (base + kl) * p.ldv + (int64_t)h * hd;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            if (d < hd) acc[j] += wgt * vrow[d];
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        if (d < hd) {
            ok = ok && isfinite(acc[j]);
            orow[d] = acc[j];
        }
    }
    if (!ok) raise_flag(p.flag, FLAG_NONFINITE);
}

hipError_t launch_audio_attention(const AudioAttnArgs &a, hipStream_t s) {
    if (a.rows <= 0) return hipSuccess;
    if (a.head_dim > 256 || a.context > 64) return hipErrorInvalidValue;
    const int64_t waves = a.rows * a.heads;
    hipLaunchKernelGGL(audio_attn_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---- light convolution: causal depthwise conv + clamp + RMSNorm + SiLU -------
// One wave per row; taps ascend from row - (K - 1), rows before the clip's
// first row are skipped (audio.rs:1490-1503). dw is [width, K].
template <int NC>
__global__ __launch_bounds__(256) void lconv_kernel(const float *__restrict__ gated,
                                                    const float *__restrict__ dw, int K,
                                                    const int32_t *__restrict__ pos, float clip,
                                                    const float *__restrict__ w, float *__restrict__ out,
                                                    int64_t rows, int width, float eps, int *flag) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int il = pos[row];
    const int nv = width >> 2;
    f32x4 v[NC];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            for (int tap = 0; tap < K; ++tap) {
                const int src = il - (K - 1) + tap;
                if (src < 0) continue;
                const f32x4 g = ((const f32x4 *)(gated + (row - il + src) * width))[i];
                const int col = 4 * i;
                acc.x += g.x * dw[(col + 0) * K + tap];
                acc.y += g.y * dw[(col + 1) * K + tap];
                acc.z += g.z * dw[(col + 2) * K + tap];
                acc.w += g.w * dw[(col + 3) * K + tap];
            }
            v[c] = clamp4(acc, -clip, clip);
            ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
        }
    }
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, width, eps);
    bool ok = isfinite(ss);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            f32x4 y = v[c] * inv * ((const f32x4 *)w)[i];
            y.x = silu_ref(y.x);
            y.y = silu_ref(y.y);
            y.z = silu_ref(y.z);
            y.w = silu_ref(y.w);
            ok = ok && finite4(y);
            ((f32x4 *)(out + row * width))[i] = y;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_lconv(const float *gated, const float *dw, int K, const int32_t *pos, float clip,
                        const float *w, float *out, int64_t rows, int width, float eps, int *flag,
                        hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (width % 4 || width > 2048) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4));
#define LC_LAUNCH(NC)                                                                           \
    hipLaunchKernelGGL(lconv_kernel<NC>, grid, dim3(256), 0, s, gated, dw, K, pos, clip, w, out, \
                       rows, width, eps, flag)
    switch ((width + 255) / 256) {
        case 1: LC_LAUNCH(1); break;
        case 2: LC_LAUNCH(2); break;
        case 3: LC_LAUNCH(3); break;
        case 4: LC_LAUNCH(4); break;
        case 5: case 6: LC_LAUNCH(6); break;
        default: LC_LAUNCH(8); break;
    }
#undef LC_LAUNCH
    return hipGetLastError();
}

// ---- unscaled RMSNorm of the valid rows, compacted ------------------------
// out[j] = x[idx[j]] * rms_inverse(x[idx[j]]); one wave per output row.
template <int NC>
__global__ __launch_bounds__(256) void compact_rms_kernel(const float *__restrict__ x,
                                                          const int32_t *__restrict__ idx,
                                                          float *__restrict__ out, int64_t rows,
                                                          int width, float eps, int *flag) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nv = width >> 2;
    const f32x4 *xr = (const f32x4 *)(x + (int64_t)idx[row] * width);
    f32x4 v[NC];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            v[c] = xr[i];
            ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
        }
    }
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, width, eps);
    bool ok = isfinite(ss);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            const f32x4 y = v[c] * inv;
            ok = ok && finite4(y);
            ((f32x4 *)(out + row * width))[i] = y;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_compact_rms(const float *x, const int32_t *idx, float *out, int64_t rows,
                              int width, float eps, int *flag, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (width % 4 || width > 2048) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4));
#define CR_LAUNCH(NC) \
    hipLaunchKernelGGL(compact_rms_kernel<NC>, grid, dim3(256), 0, s, x, idx, out, rows, width, eps, flag)
    switch ((width + 255) / 256) {
        case 1: CR_LAUNCH(1); break;
        case 2: CR_LAUNCH(2); break;
        case 3: CR_LAUNCH(3); break;
        case 4: CR_LAUNCH(4); break;
        case 5: case 6: CR_LAUNCH(6); break;
        default: CR_LAUNCH(8); break;
    }
#undef CR_LAUNCH
    return hipGetLastError();
}

}  // namespace svl
