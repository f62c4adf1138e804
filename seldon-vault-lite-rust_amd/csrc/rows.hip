// Bandwidth-bound row kernels of the encoder: RMSNorm variants fused with the
// residual add and layer scalar, the embedding gather, the per-head Q/K/V
// norm + RoPE, masked mean pooling with L2 / Matryoshka normalisation, and
// the elementwise seam kernels.
//
// All row kernels run one wave64 per row: a 768-float hidden row is 3 float4
// per lane, read once, reduced with cross-lane shuffles, and written once,
// so each kernel moves exactly its algorithmic bytes through HBM.
#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

constexpr int ROW_CHUNKS = 8;  // register-resident rows up to 8 * 256 floats

// Launch a kernel templated on the number of 256-float chunks per row.
#define SVL_DISPATCH_NC(nc, KERNEL, grid, ...)                                                  \
    switch (nc) {                                                                             \
        case 1: hipLaunchKernelGGL(KERNEL<1>, grid, dim3(256), 0, __VA_ARGS__); break;        \
        case 2: hipLaunchKernelGGL(KERNEL<2>, grid, dim3(256), 0, __VA_ARGS__); break;        \
        case 3: hipLaunchKernelGGL(KERNEL<3>, grid, dim3(256), 0, __VA_ARGS__); break;        \
        case 4: hipLaunchKernelGGL(KERNEL<4>, grid, dim3(256), 0, __VA_ARGS__); break;        \
        case 5: hipLaunchKernelGGL(KERNEL<5>, grid, dim3(256), 0, __VA_ARGS__); break;        \
        case 6: hipLaunchKernelGGL(KERNEL<6>, grid, dim3(256), 0, __VA_ARGS__); break;        \
        case 7: hipLaunchKernelGGL(KERNEL<7>, grid, dim3(256), 0, __VA_ARGS__); break;        \
        default: hipLaunchKernelGGL(KERNEL<8>, grid, dim3(256), 0, __VA_ARGS__); break;       \
    }

// The same with a second, boolean template argument B.
#define SVL_DISPATCH_NC_B(nc, KERNEL, B, grid, ...)                                             \
    switch (nc) {                                                                             \
        case 1: hipLaunchKernelGGL((KERNEL<1, B>), grid, dim3(256), 0, __VA_ARGS__); break;   \
        case 2: hipLaunchKernelGGL((KERNEL<2, B>), grid, dim3(256), 0, __VA_ARGS__); break;   \
        case 3: hipLaunchKernelGGL((KERNEL<3, B>), grid, dim3(256), 0, __VA_ARGS__); break;   \
        case 4: hipLaunchKernelGGL((KERNEL<4, B>), grid, dim3(256), 0, __VA_ARGS__); break;   \
        case 5: hipLaunchKernelGGL((KERNEL<5, B>), grid, dim3(256), 0, __VA_ARGS__); break;   \
        case 6: hipLaunchKernelGGL((KERNEL<6, B>), grid, dim3(256), 0, __VA_ARGS__); break;   \
        case 7: hipLaunchKernelGGL((KERNEL<7, B>), grid, dim3(256), 0, __VA_ARGS__); break;   \
        default: hipLaunchKernelGGL((KERNEL<8, B>), grid, dim3(256), 0, __VA_ARGS__); break;  \
    }

// Row kernels whose launch covers fewer rows than this load every operand of
// a row before its arithmetic (LOAD_FIRST below); larger launches keep the
// load order that holds fewer registers per wave.
constexpr int64_t LOAD_FIRST_MAX_ROWS = 4096;

// ---- RMSNorm rows (kernels.rs:727-857) ------------------------------------

// Register-resident variant: width % 4 == 0 and width <= 2048.
template <int NC>
__global__ __launch_bounds__(256) void rms_rows_kernel(const float *__restrict__ x,
                                                       const float *__restrict__ w,
                                                       float *__restrict__ out, int64_t rows,
                                                       int width, float eps, int *flag) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nv = width >> 2;
    const f32x4 *xr = (const f32x4 *)(x + row * width);
    // the row and the weights loaded together (chunks past the width load
    // its last chunk and take no part)
    f32x4 v[NC], wv[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = min(lane + 64 * c, nv - 1);
        v[c] = xr[i];
        if (w) wv[c] = ((const f32x4 *)w)[i];
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
        if (lane + 64 * c < nv)
            ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, width, eps);
    bool ok = isfinite(ss);
    f32x4 *orow = (f32x4 *)(out + row * width);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            f32x4 y = v[c] * inv;
            if (w) y = y * wv[c];
            ok = ok && finite4(y);
            orow[i] = y;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

// Any width: two passes over the row.
__global__ __launch_bounds__(256) void rms_rows_generic_kernel(const float *__restrict__ x,
                                                               const float *__restrict__ w,
                                                               float *__restrict__ out,
                                                               int64_t rows, int width, float eps,
                                                               int *flag) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + row * width;
    float ss = 0.f;
    for (int i = lane; i < width; i += 64) ss += xr[i] * xr[i];
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, width, eps);
    bool ok = isfinite(ss);
    for (int i = lane; i < width; i += 64) {
        float y = xr[i] * inv;
        if (w) y = y * w[i];
        ok = ok && isfinite(y);
        out[row * width + i] = y;
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_rms_rows(const float *x, const float *w, float *out, int64_t rows, int width,
                           float eps, int *flag, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + 3) / 4));
    const bool vec = width > 0 && width % 4 == 0 && width <= 256 * ROW_CHUNKS &&
                     (uintptr_t)x % 16 == 0 &&
                     (uintptr_t)out % 16 == 0 && (!w || (uintptr_t)w % 16 == 0);
    if (vec) {
        SVL_DISPATCH_NC((width + 255) / 256, rms_rows_kernel, grid, s, x, w, out, rows, width, eps,
                        flag);
    } else
        hipLaunchKernelGGL(rms_rows_generic_kernel, grid, dim3(256), 0, s, x, w, out, rows, width,
                           eps, flag);
    return hipGetLastError();
}

// ---- residual + post-norm (+ layer scalar) (+ next pre-norm) ---------------
// text.rs:424-433 / 465-472 / 502-513 and the following rms_norm_rows:
//   h = (res + rms(x, w1)) * scale;  n = rms(h, w2)
// (res + y) * scale rounds exactly like add() then the scalar multiply.
// h_out may alias res (in-place residual update): each lane reads its
// elements of res before writing the same elements of h_out.
//
// Two load orders, one arithmetic. LOAD_FIRST loads every operand of the
// row before any arithmetic (chunks past the width load its last chunk and
// take no part): one memory round trip where the other order takes one per
// chunk and operand, which sets the time of a launch over a few hundred rows
// (the 1 x 128-token forward's 72 launches: 5.1 against 3.6 us). Launches
// of many rows take the other order, whose waves hold fewer registers: with
// the other row groups' GEMMs on the same CUs the three-group T2 step took
// 39.50 against 39.36 ms with every launch loading first.
template <int NC, bool LOAD_FIRST>
__global__ __launch_bounds__(256) void resnorm_kernel(
    const float *__restrict__ x, const float *__restrict__ w1, const float *res, float *h_out,
    const float *__restrict__ w2, float *__restrict__ n_out,
    float scale, int64_t rows, int width, float eps, int *flag) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nv = width >> 2;
    const f32x4 *xr = (const f32x4 *)(x + row * width);
    const f32x4 *rr = (const f32x4 *)(res + row * width);
    f32x4 v[NC], rv[NC], w1v[NC], w2v[NC];
    float ss = 0.f;
    if constexpr (LOAD_FIRST) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int i = min(lane + 64 * c, nv - 1);
            v[c] = xr[i];
            rv[c] = rr[i];
            w1v[c] = ((const f32x4 *)w1)[i];
            if (w2) w2v[c] = ((const f32x4 *)w2)[i];
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (lane + 64 * c < nv)
                ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
    } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int i = lane + 64 * c;
            if (i < nv) {
                v[c] = xr[i];
                ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
            }
        }
    }
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, width, eps);
    bool ok = isfinite(ss);
    float ss2 = 0.f;
    f32x4 *hrow = (f32x4 *)(h_out + row * width);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            if constexpr (!LOAD_FIRST) {
                w1v[c] = ((const f32x4 *)w1)[i];
                rv[c] = rr[i];
            }
            const f32x4 y = v[c] * inv * w1v[c];
            f32x4 hv = (rv[c] + y) * scale;
            ok = ok && finite4(hv);
            hrow[i] = hv;
            v[c] = hv;
            ss2 += hv.x * hv.x + hv.y * hv.y + hv.z * hv.z + hv.w * hv.w;
        }
    }
    if (w2) {
        ss2 = wave_sum(ss2);
        const float inv2 = rms_inverse(ss2, width, eps);
        f32x4 *nrow = (f32x4 *)(n_out + row * width);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int i = lane + 64 * c;
            if (i < nv) {
                if constexpr (!LOAD_FIRST) w2v[c] = ((const f32x4 *)w2)[i];
                const f32x4 y = v[c] * inv2 * w2v[c];
                ok = ok && finite4(y);
                nrow[i] = y;
            }
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_resnorm(const float *x, const float *w1, const float *res, float *h_out,
                          const float *w2, float *n_out, float scale, int64_t rows, int width,
                          float eps, int *flag, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (width <= 0 || width % 4 != 0 || width > 256 * ROW_CHUNKS) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (rows < LOAD_FIRST_MAX_ROWS) {
        SVL_DISPATCH_NC_B((width + 255) / 256, resnorm_kernel, true, grid, s, x, w1, res, h_out,
                          w2, n_out, scale, rows, width, eps, flag);
    } else {
        SVL_DISPATCH_NC_B((width + 255) / 256, resnorm_kernel, false, grid, s, x, w1, res, h_out,
                          w2, n_out, scale, rows, width, eps, flag);
    }
    return hipGetLastError();
}

// ---- embedding gather (text.rs:209-275) + first input_layernorm ------------
template <int NC>
__global__ __launch_bounds__(256) void gather_kernel(
    const uint32_t *__restrict__ ids, const float *__restrict__ table, int64_t vocab,
    const int32_t *__restrict__ featmap, const float *__restrict__ feats, float scale,
    const float *__restrict__ w_in, float *__restrict__ h, float *__restrict__ n, int64_t tokens,
    int width, float eps, int *flag) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= tokens) return;
    const int nv = width >> 2;
    const int fi = featmap ? featmap[t] : -1;
    const f32x4 *src;
    float mul = scale;
    if (fi >= 0) {
        src = (const f32x4 *)(feats + (int64_t)fi * width);
        mul = 1.0f;
    } else {
        uint32_t id = ids[t];
        if (id >= (uint64_t)vocab) {
            if (lane == 0) raise_flag(flag, FLAG_BAD_TOKEN);
            id = 0;
        }
        src = (const f32x4 *)(table + (int64_t)id * width);
    }
    // the row's chunks and the norm weights loaded together (chunks past the
    // width load its last chunk and take no part)
    f32x4 v[NC], wv[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = min(lane + 64 * c, nv - 1);
        v[c] = src[i];
        wv[c] = ((const f32x4 *)w_in)[i];
    }
    float ss = 0.f;
    bool ok = true;
    f32x4 *hrow = (f32x4 *)(h + t * width);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            f32x4 e = v[c];
            if (fi < 0) e = e * mul;
            v[c] = e;
            ok = ok && finite4(e);
            hrow[i] = e;
            ss += e.x * e.x + e.y * e.y + e.z * e.z + e.w * e.w;
        }
    }
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, width, eps);
    f32x4 *nrow = (f32x4 *)(n + t * width);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            const f32x4 y = v[c] * inv * wv[c];
            ok = ok && finite4(y);
            nrow[i] = y;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_gather(const uint32_t *ids, const float *table, int64_t vocab,
                         const int32_t *featmap, const float *feats, float scale,
                         const float *w_in, float *h, float *n, int64_t tokens, int width,
                         float eps, int *flag, hipStream_t s) {
    if (tokens <= 0) return hipSuccess;
    if (width <= 0 || width % 4 != 0 || width > 256 * ROW_CHUNKS) return hipErrorInvalidValue;
    SVL_DISPATCH_NC((width + 255) / 256, gather_kernel, dim3((unsigned)((tokens + 3) / 4)), s, ids,
                    table, vocab, featmap, feats, scale, w_in, h, n, tokens, width, eps, flag);
    return hipGetLastError();
}

// ---- per-head Q/K norm + RoPE, V unscaled norm (text.rs:370-405) -----------
// One wave per head row of the fused QKV output [T, nh*hd + 2*nkv*hd]. The
// normalised row is staged in LDS so each lane can rotate the pair
// (j, j + hd/2) of rotate-half RoPE (kernels.rs:974-981).
constexpr int QKV_MAX_HD = 1024;

__global__ __launch_bounds__(256) void qkv_post_kernel(
    float *__restrict__ qkv, int64_t ld, int64_t tokens, int nh, int nkv, int hd,
    const float *__restrict__ qn, const float *__restrict__ kn, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int32_t *__restrict__ pos, float eps, int *flag) {
    __shared__ float stage[4][QKV_MAX_HD];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int per_tok = nh + 2 * nkv;
    const int64_t hr = (int64_t)blockIdx.x * 4 + wave;
    if (hr >= tokens * per_tok) return;
    const int64_t t = hr / per_tok;
    const int k = (int)(hr - t * per_tok);
    // kind 0: q head, 1: k head, 2: v head
    const int kind = k < nh ? 0 : (k < nh + nkv ? 1 : 2);
    float *row = qkv + t * ld + (int64_t)k * hd;  // q, k, v heads are contiguous in this order
    const float *w = kind == 0 ? qn : (kind == 1 ? kn : nullptr);
    float ss = 0.f;
    for (int i = lane; i < hd; i += 64) ss += row[i] * row[i];
    ss = wave_sum(ss);
    const float inv = rms_inverse(ss, hd, eps);
    bool ok = isfinite(ss);
    if (kind == 2) {
        for (int i = lane; i < hd; i += 64) {
            const float y = row[i] * inv;
            ok = ok && isfinite(y);
            row[i] = y;
        }
    } else {
        float *st = stage[wave];
        for (int i = lane; i < hd; i += 64) st[i] = row[i] * inv * w[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int half = hd >> 1;
        const int64_t tab = (int64_t)pos[t] * half;
        for (int j = lane; j < half; j += 64) {
            const float first = st[j], second = st[j + half];
            const float c = cos_t[tab + j], sn = sin_t[tab + j];
            const float a = first * c - second * sn;
            const float b = first * sn + second * c;
            ok = ok && isfinite(a) && isfinite(b);
            row[j] = a;
            row[j + half] = b;
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

// head_dim 256 fast path: one wave per token, two head rows per wave
// instruction. Lane l works on row 2 i + l / 32 of the token, elements
// [4 (l % 32), +4) and [128 + 4 (l % 32), +4): the rotate-half partner of
// each element (j and j + 128) sits in the same lane, and each row's norm is
// a 32-lane reduction.
template <int PAIRS, bool LOAD_FIRST>
__global__ __launch_bounds__(256) void qkv_post256_kernel(
    float *__restrict__ qkv, int64_t ld, int64_t tokens, int nh, int nkv,
    const float *__restrict__ qn, const float *__restrict__ kn, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int32_t *__restrict__ pos, float eps, int *flag) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= tokens) return;
    const int per_tok = nh + 2 * nkv;
    const int h = lane >> 5, l32 = lane & 31;
    f32x4 *row = (f32x4 *)(qkv + t * ld) + 64 * h + l32;  // row h of the token
    f32x4 x[PAIRS][2], wq0, wq1, wk0, wk1, c, sn;
    float ss[PAIRS];
    if constexpr (LOAD_FIRST) {
        // Every operand is loaded before any arithmetic (rows past the
        // token's last load that row and take no part): two memory round
        // trips, the position and then its table rows, instead of one per
        // row pair (the load orders of resnorm_kernel).
        const int64_t tab = (int64_t)pos[t] * 128 + 4 * l32;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            const f32x4 *src =
                (const f32x4 *)(qkv + t * ld) + 64 * min(2 * i + h, per_tok - 1) + l32;
            x[i][0] = src[0];
            x[i][1] = src[32];
        }
        wq0 = ((const f32x4 *)qn)[l32];
        wq1 = ((const f32x4 *)qn)[l32 + 32];
        wk0 = ((const f32x4 *)kn)[l32];
        wk1 = ((const f32x4 *)kn)[l32 + 32];
        c = *(const f32x4 *)(cos_t + tab);
        sn = *(const f32x4 *)(sin_t + tab);
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            ss[i] = 0.f;
            if (2 * i + h < per_tok)
                ss[i] = x[i][0].x * x[i][0].x + x[i][0].y * x[i][0].y + x[i][0].z * x[i][0].z +
                        x[i][0].w * x[i][0].w + x[i][1].x * x[i][1].x + x[i][1].y * x[i][1].y +
                        x[i][1].z * x[i][1].z + x[i][1].w * x[i][1].w;
        }
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) ss[i] = group_reduce<32, false>(ss[i]);
    } else {
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            ss[i] = 0.f;
            if (2 * i + h < per_tok) {
                x[i][0] = row[128 * i];
                x[i][1] = row[128 * i + 32];
                ss[i] = x[i][0].x * x[i][0].x + x[i][0].y * x[i][0].y + x[i][0].z * x[i][0].z +
                        x[i][0].w * x[i][0].w + x[i][1].x * x[i][1].x + x[i][1].y * x[i][1].y +
                        x[i][1].z * x[i][1].z + x[i][1].w * x[i][1].w;
            }
        }
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) ss[i] = group_reduce<32, false>(ss[i]);
        wq0 = ((const f32x4 *)qn)[l32];
        wq1 = ((const f32x4 *)qn)[l32 + 32];
        wk0 = ((const f32x4 *)kn)[l32];
        wk1 = ((const f32x4 *)kn)[l32 + 32];
        const int64_t tab = (int64_t)pos[t] * 128 + 4 * l32;
        c = *(const f32x4 *)(cos_t + tab);
        sn = *(const f32x4 *)(sin_t + tab);
    }
    bool ok = true;
#pragma unroll
    for (int i = 0; i < PAIRS; ++i) {
        const int k = 2 * i + h;
        if (k >= per_tok) continue;
        ok = ok && isfinite(ss[i]);
        const float inv = rms_inverse(ss[i], 256, eps);
        if (k >= nh + nkv) {  // value head: unscaled norm, no rotation
            const f32x4 y0 = x[i][0] * inv, y1 = x[i][1] * inv;
            ok = ok && finite4(y0) && finite4(y1);
            row[128 * i] = y0;
            row[128 * i + 32] = y1;
            continue;
        }
        const f32x4 first = x[i][0] * inv * (k < nh ? wq0 : wk0);
        const f32x4 second = x[i][1] * inv * (k < nh ? wq1 : wk1);
        const f32x4 a = first * c - second * sn;
        const f32x4 b = first * sn + second * c;
        ok = ok && finite4(a) && finite4(b);
        row[128 * i] = a;
        row[128 * i + 32] = b;
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

// head_dim 512 fast path: one wave per token. Lane l holds elements
// [4l, 4l+4) and [256+4l, 256+4l+4) of every head row, so the rotate-half
// partner of each element (j and j + 256) sits in the same lane.
template <int ROWS, bool LOAD_FIRST>
__global__ __launch_bounds__(256) void qkv_post512_kernel(
    float *__restrict__ qkv, int64_t ld, int64_t tokens, int nh, int nkv,
    const float *__restrict__ qn, const float *__restrict__ kn, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int32_t *__restrict__ pos, float eps, int *flag) {
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= tokens) return;
    const int per_tok = nh + 2 * nkv;
    f32x4 *row = (f32x4 *)(qkv + t * ld) + lane;
    f32x4 x[ROWS][2], wq0, wq1, wk0, wk1, c, sn;
    float ss[ROWS];
    if constexpr (LOAD_FIRST) {
        // every operand loaded before any arithmetic, as in qkv_post256_kernel
        const int64_t tab = (int64_t)pos[t] * 256 + 4 * lane;
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
            const int kr = min(k, per_tok - 1);
            x[k][0] = row[128 * kr];
            x[k][1] = row[128 * kr + 64];
        }
        wq0 = ((const f32x4 *)qn)[lane];
        wq1 = ((const f32x4 *)qn)[lane + 64];
        wk0 = ((const f32x4 *)kn)[lane];
        wk1 = ((const f32x4 *)kn)[lane + 64];
        c = *(const f32x4 *)(cos_t + tab);
        sn = *(const f32x4 *)(sin_t + tab);
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
            ss[k] = 0.f;
            if (k < per_tok)
                ss[k] = x[k][0].x * x[k][0].x + x[k][0].y * x[k][0].y + x[k][0].z * x[k][0].z +
                        x[k][0].w * x[k][0].w + x[k][1].x * x[k][1].x + x[k][1].y * x[k][1].y +
                        x[k][1].z * x[k][1].z + x[k][1].w * x[k][1].w;
        }
#pragma unroll
        for (int k = 0; k < ROWS; ++k)
            if (k < per_tok) ss[k] = wave_sum(ss[k]);
    } else {
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
            if (k < per_tok) {
                x[k][0] = row[128 * k];
                x[k][1] = row[128 * k + 64];
                ss[k] = x[k][0].x * x[k][0].x + x[k][0].y * x[k][0].y + x[k][0].z * x[k][0].z +
                        x[k][0].w * x[k][0].w + x[k][1].x * x[k][1].x + x[k][1].y * x[k][1].y +
                        x[k][1].z * x[k][1].z + x[k][1].w * x[k][1].w;
            }
        }
#pragma unroll
        for (int k = 0; k < ROWS; ++k)
            if (k < per_tok) ss[k] = wave_sum(ss[k]);
        wq0 = ((const f32x4 *)qn)[lane];
        wq1 = ((const f32x4 *)qn)[lane + 64];
        wk0 = ((const f32x4 *)kn)[lane];
        wk1 = ((const f32x4 *)kn)[lane + 64];
        const int64_t tab = (int64_t)pos[t] * 256 + 4 * lane;
        c = *(const f32x4 *)(cos_t + tab);
        sn = *(const f32x4 *)(sin_t + tab);
    }
    bool ok = true;
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
        if (k >= per_tok) continue;
        ok = ok && isfinite(ss[k]);
        const float inv = rms_inverse(ss[k], 512, eps);
        if (k >= nh + nkv) {  // value head: unscaled norm, no rotation
            const f32x4 y0 = x[k][0] * inv, y1 = x[k][1] * inv;
            ok = ok && finite4(y0) && finite4(y1);
            row[128 * k] = y0;
            row[128 * k + 64] = y1;
            continue;
        }
        const f32x4 first = x[k][0] * inv * (k < nh ? wq0 : wk0);
        const f32x4 second = x[k][1] * inv * (k < nh ? wq1 : wk1);
        const f32x4 a = first * c - second * sn;
        const f32x4 b = first * sn + second * c;
        ok = ok && finite4(a) && finite4(b);
        row[128 * k] = a;
        row[128 * k + 64] = b;
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_qkv_post(float *qkv, int64_t ld, int64_t tokens, int nh, int nkv, int hd,
                           const float *qn, const float *kn, const float *cos_t,
                           const float *sin_t, const int32_t *pos, float eps, int *flag,
                           hipStream_t s) {
    const int64_t head_rows = tokens * (nh + 2 * nkv);
    if (head_rows <= 0) return hipSuccess;
    if (hd > QKV_MAX_HD || hd % 2) return hipErrorInvalidValue;
    const bool aligned = ld % 4 == 0 && (uintptr_t)qkv % 16 == 0;
    if (hd == 256 && aligned && nh + 2 * nkv <= 8) {
        const dim3 grid((unsigned)((tokens + 3) / 4));
        const bool first = tokens < LOAD_FIRST_MAX_ROWS;
        if (nh + 2 * nkv <= 6) {
            if (first)
                hipLaunchKernelGGL((qkv_post256_kernel<3, true>), grid, dim3(256), 0, s, qkv, ld,
                                   tokens, nh, nkv, qn, kn, cos_t, sin_t, pos, eps, flag);
            else
                hipLaunchKernelGGL((qkv_post256_kernel<3, false>), grid, dim3(256), 0, s, qkv, ld,
                                   tokens, nh, nkv, qn, kn, cos_t, sin_t, pos, eps, flag);
        } else {
            if (first)
                hipLaunchKernelGGL((qkv_post256_kernel<4, true>), grid, dim3(256), 0, s, qkv, ld,
                                   tokens, nh, nkv, qn, kn, cos_t, sin_t, pos, eps, flag);
            else
                hipLaunchKernelGGL((qkv_post256_kernel<4, false>), grid, dim3(256), 0, s, qkv, ld,
                                   tokens, nh, nkv, qn, kn, cos_t, sin_t, pos, eps, flag);
        }
        return hipGetLastError();
    }
    if (hd == 512 && aligned && nh + 2 * nkv <= 6) {
        const dim3 grid((unsigned)((tokens + 3) / 4));
        if (tokens < LOAD_FIRST_MAX_ROWS)
            hipLaunchKernelGGL((qkv_post512_kernel<6, true>), grid, dim3(256), 0, s, qkv, ld,
                               tokens, nh, nkv, qn, kn, cos_t, sin_t, pos, eps, flag);
        else
            hipLaunchKernelGGL((qkv_post512_kernel<6, false>), grid, dim3(256), 0, s, qkv, ld,
                               tokens, nh, nkv, qn, kn, cos_t, sin_t, pos, eps, flag);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(qkv_post_kernel, dim3((unsigned)((head_rows + 3) / 4)), dim3(256), 0, s,
                       qkv, ld, tokens, nh, nkv, hd, qn, kn, cos_t, sin_t, pos, eps, flag);
    return hipGetLastError();
}

// RoPE alone on [T, heads, hd] (kernels.rs:936-988); table row t = position t.
__global__ __launch_bounds__(256) void rope_kernel(float *__restrict__ x, int64_t tokens,
                                                   int heads, int hd,
                                                   const float *__restrict__ cos_t,
                                                   const float *__restrict__ sin_t, int *flag) {
    const int64_t hr = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (hr >= tokens * heads) return;
    const int64_t t = hr / heads;
    float *row = x + hr * hd;
    const int half = hd >> 1;
    bool ok = true;
    for (int j = lane; j < half; j += 64) {
        const float first = row[j], second = row[j + half];
        const float c = cos_t[t * half + j], sn = sin_t[t * half + j];
        const float a = first * c - second * sn;
        const float b = first * sn + second * c;
        ok = ok && isfinite(a) && isfinite(b);
        row[j] = a;
        row[j + half] = b;
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_rope(float *x, int64_t tokens, int heads, int hd, const float *cos_t,
                       const float *sin_t, int *flag, hipStream_t s) {
    const int64_t rows = tokens * heads;
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, x, tokens,
                       heads, hd, cos_t, sin_t, flag);
    return hipGetLastError();
}

// ---- token positions from row offsets --------------------------------------
__global__ __launch_bounds__(256) void positions_kernel(const int64_t *__restrict__ offsets,
                                                        int32_t *__restrict__ pos,
                                                        int32_t *__restrict__ rowlen) {
    const int r = blockIdx.x;
    const int64_t a = offsets[r], b = offsets[r + 1];
    for (int64_t t = a + threadIdx.x; t < b; t += 256) {
        pos[t] = (int32_t)(t - a);
        if (rowlen) rowlen[t] = (int32_t)(b - a);
    }
}

hipError_t launch_positions(const int64_t *offsets, int batch, int32_t *pos, int32_t *rowlen,
                            hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    hipLaunchKernelGGL(positions_kernel, dim3(batch), dim3(256), 0, s, offsets, pos, rowlen);
    return hipGetLastError();
}

// ---- masked mean pool + L2 + Matryoshka (kernels.rs:882-927) ---------------
// pool_sum_kernel: one 64-lane workgroup per (row, 64 columns); each lane
// sums its column over the row's tokens in token order and multiplies by
// 1/len: the same operations in the same order as mean_pool_scalar, so
// pooled is bit-identical for identical projected inputs. Loads are issued
// 32 (then 8) tokens ahead of the additions, so a row costs a few memory
// round trips rather than one per eight tokens.
// pool_norm_kernel: one workgroup per row: L2 normalisation and the
// Matryoshka truncations, each renormalised.
constexpr int POOL_MAX_WIDTH = 4096;

__device__ float block_sum_256(float v, float *red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(64) void pool_sum_kernel(const float *__restrict__ proj, int width,
                                                      const int64_t *__restrict__ offsets,
                                                      float *__restrict__ pooled, int *flag) {
    const int r = blockIdx.x;
    const int c = blockIdx.y * 64 + threadIdx.x;
    if (c >= width) return;
    const int64_t a = offsets[r], b = offsets[r + 1];
    const float *src = proj + a * width + c;
    const int64_t n = b - a;
    float acc = 0.f;
    int64_t t = 0;
    // 32 loads in flight per round trip: a 128-token row takes four
    for (; t + 32 <= n; t += 32) {
        float v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = src[(t + u) * width];
#pragma unroll
        for (int u = 0; u < 32; ++u) acc += v[u];
    }
    for (; t + 8 <= n; t += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = src[(t + u) * width];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; t < n; ++t) acc += src[t * width];
    acc *= 1.0f / (float)n;
    if (!isfinite(acc)) raise_flag(flag, FLAG_NONFINITE);
    pooled[(int64_t)r * width + c] = acc;
}

__global__ __launch_bounds__(256) void pool_norm_kernel(const float *__restrict__ pooled, int width,
                                                        const int32_t *__restrict__ dims,
                                                        int n_dims, int dims_total,
                                                        float *__restrict__ normalized,
                                                        float *__restrict__ trunc_out, int *flag) {
    __shared__ float nv[POOL_MAX_WIDTH];
    __shared__ float red[4];
    const int r = blockIdx.x;
    float ss = 0.f;
    for (int c = threadIdx.x; c < width; c += 256) {
        const float v = pooled[(int64_t)r * width + c];
        nv[c] = v;
        ss += v * v;
    }
    ss = block_sum_256(ss, red);
    bool ok = isfinite(ss) && ss > 0.f;
    const float inv = 1.0f / sqrtf(ss);
    for (int c = threadIdx.x; c < width; c += 256) {
        const float y = nv[c] * inv;
        nv[c] = y;
        if (normalized) normalized[(int64_t)r * width + c] = y;
    }
    __syncthreads();
    int off = 0;
    for (int d = 0; d < n_dims; ++d) {
        const int dim = dims[d];
        float s2 = 0.f;
        for (int c = threadIdx.x; c < dim; c += 256) s2 += nv[c] * nv[c];
        s2 = block_sum_256(s2, red);
        const float inv_d = 1.0f / sqrtf(s2);
        ok = ok && isfinite(s2) && s2 > 0.f;
        if (trunc_out)
            for (int c = threadIdx.x; c < dim; c += 256)
                trunc_out[(int64_t)r * dims_total + off + c] = nv[c] * inv_d;
        off += dim;
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_pool(const float *proj, int width, const int64_t *offsets, int batch,
                       const int32_t *dims, int n_dims, int dims_total, float *pooled,
                       float *normalized, float *trunc_out, int *flag, hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    if (width > POOL_MAX_WIDTH || !pooled) return hipErrorInvalidValue;
    hipLaunchKernelGGL(pool_sum_kernel, dim3(batch, (width + 63) / 64), dim3(64), 0, s, proj,
                       width, offsets, pooled, flag);
    if (!normalized && !trunc_out) return hipGetLastError();
    return launch_pool_norm(pooled, width, batch, dims, n_dims, dims_total, normalized, trunc_out,
                            flag, s);
}

hipError_t launch_pool_norm(const float *pooled, int width, int batch, const int32_t *dims,
                            int n_dims, int dims_total, float *normalized, float *trunc_out,
                            int *flag, hipStream_t s) {
    if (batch <= 0) return hipSuccess;
    if (width > POOL_MAX_WIDTH) return hipErrorInvalidValue;
    hipLaunchKernelGGL(pool_norm_kernel, dim3(batch), dim3(256), 0, s, pooled, width, dims, n_dims,
                       dims_total, normalized, trunc_out, flag);
    return hipGetLastError();
}

// ---- elementwise seam kernels ----------------------------------------------
__global__ __launch_bounds__(256) void gelu_kernel(const float *x, float *y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = gelu_tanh(x[i]);
}
__global__ __launch_bounds__(256) void geglu_kernel(const float *g, const float *u, float *y,
                                                    int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = gelu_tanh(g[i]) * u[i];
}
__global__ __launch_bounds__(256) void add_kernel(const float *a, const float *b, float *y,
                                                  int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = a[i] + b[i];
}
__global__ __launch_bounds__(256) void finite_kernel(const float *x, int64_t n, int *flag) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n && !isfinite(x[i])) raise_flag(flag, FLAG_NONFINITE);
}

static dim3 grid1d(int64_t n) { return dim3((unsigned)((n + 255) / 256)); }

hipError_t launch_gelu(const float *x, float *y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(gelu_kernel, grid1d(n), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}
hipError_t launch_geglu(const float *g, const float *u, float *y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(geglu_kernel, grid1d(n), dim3(256), 0, s, g, u, y, n);
    return hipGetLastError();
}
hipError_t launch_add(const float *a, const float *b, float *y, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(add_kernel, grid1d(n), dim3(256), 0, s, a, b, y, n);
    return hipGetLastError();
}
hipError_t launch_finite_check(const float *x, int64_t n, int *flag, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(finite_kernel, grid1d(n), dim3(256), 0, s, x, n, flag);
    return hipGetLastError();
}

}  // namespace svl
