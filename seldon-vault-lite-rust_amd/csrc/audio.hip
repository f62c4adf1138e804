// Row kernels of the audio tower (src/model/audio.rs:981-1690). The
// projections are the shared GEMM with the clipped-linear epilogues; what is
// specific to the tower lives here:
//  * the two stride-2 3x3 subsampling convolutions, each with its per-position
//    LayerNorm (weight, no bias) and ReLU (audio.rs:1136-1255, 1290-1322):
//    the first direct, the second as an implicit-im2col MFMA GEMM
//    (launch_gemm_conv) followed by the LayerNorm + ReLU kernel here;
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
// One workgroup per layer-0 row: the three mel rows it reads (zero where the
// tap is outside the clip, masked or past the 128 bins) and the 3x3 weights
// go to LDS; four threads per output frequency, each with CPT consecutive
// channels. Each channel sums its nine taps in (kernel row, kernel column)
// order; the LayerNorm sums reduce over the four threads.
constexpr int SSCP_TAPS_W = MEL_BINS + 2;  // one zero column on each side

template <int CPT>
__global__ __launch_bounds__(256) void sscp_conv0_kernel(const float *__restrict__ mel,
                                                         const uint8_t *__restrict__ mask,
                                                         const SscpRow *__restrict__ rows,
                                                         const float *__restrict__ w,
                                                         const float *__restrict__ ln, int C0,
                                                         float eps, float *__restrict__ out,
                                                         int *flag) {
    __shared__ float taps[3][SSCP_TAPS_W];
    __shared__ float ws[4 * CPT * 9];
    const int64_t r = blockIdx.x;
    const SscpRow ri = rows[r];
    for (int i = threadIdx.x; i < C0 * 9; i += 256) ws[i] = w[i];
    for (int i = threadIdx.x; i < 3 * SSCP_TAPS_W; i += 256) {
        const int kt = i / SSCP_TAPS_W, x = i - kt * SSCP_TAPS_W, iff = x - 1;
        const int it = 2 * ri.t + kt - 1;
        const bool in = it >= 0 && it < ri.len && iff >= 0 && iff < MEL_BINS && mask[ri.base + it];
        taps[kt][x] = in ? mel[(int64_t)(ri.base + it) * MEL_BINS + iff] : 0.0f;
    }
    __syncthreads();
    const int f = threadIdx.x >> 2, c0 = (threadIdx.x & 3) * CPT;
    float tap[9];
#pragma unroll
    for (int kt = 0; kt < 3; ++kt)
#pragma unroll
        for (int kf = 0; kf < 3; ++kf) tap[kt * 3 + kf] = taps[kt][2 * f + kf];
    float v[CPT];
    float sum = 0.f;
    bool ok = true;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        float acc = 0.0f;
        if (c0 + j < C0) {
#pragma unroll
            for (int k = 0; k < 9; ++k) acc += tap[k] * ws[(c0 + j) * 9 + k];
            ok = ok && isfinite(acc);
            sum += acc;
        }
        v[j] = acc;
    }
    sum = group_reduce<4, false>(sum);
    const float mean = sum / (float)C0;
    float var = 0.f;
#pragma unroll
    for (int j = 0; j < CPT; ++j)
        if (c0 + j < C0) {
            const float d = v[j] - mean;
            var += d * d;
        }
    var = group_reduce<4, false>(var);
    var = var / (float)C0;
    const float inv = 1.0f / sqrtf(var + eps);
    ok = ok && isfinite(inv);
    float *o = out + (r * FREQ0 + f) * C0 + c0;
    if (CPT % 4 == 0 && C0 == 4 * CPT) {
#pragma unroll
        for (int j = 0; j < CPT; j += 4)
            *(f32x4 *)(o + j) = f32x4{fmaxf((v[j] - mean) * inv * ln[c0 + j], 0.0f),
                                      fmaxf((v[j + 1] - mean) * inv * ln[c0 + j + 1], 0.0f),
                                      fmaxf((v[j + 2] - mean) * inv * ln[c0 + j + 2], 0.0f),
                                      fmaxf((v[j + 3] - mean) * inv * ln[c0 + j + 3], 0.0f)};
    } else {
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            if (c0 + j < C0) o[j] = fmaxf((v[j] - mean) * inv * ln[c0 + j], 0.0f);
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_sscp_conv0(const float *mel, const uint8_t *mask, const SscpRow *rows,
                             int64_t n_rows, const float *w, const float *ln, int C0, float eps,
                             float *out, int *flag, hipStream_t s) {
    if (n_rows <= 0) return hipSuccess;
    if (n_rows > INT32_MAX || C0 < 1) return hipErrorInvalidValue;
    static_assert(FREQ0 * 4 == 256, "four threads per output frequency");
#define C0_LAUNCH(CPT)                                                                       \
    hipLaunchKernelGGL(sscp_conv0_kernel<CPT>, dim3((unsigned)n_rows), dim3(256), 0, s, mel, \
                       mask, rows, w, ln, C0, eps, out, flag)
    const int cpt = (C0 + 3) / 4;
    if (cpt <= 8) C0_LAUNCH(8);
    else if (cpt <= 16) C0_LAUNCH(16);
    else if (cpt <= 32) C0_LAUNCH(32);
    else if (cpt <= 64) C0_LAUNCH(64);
    else if (cpt <= 128) C0_LAUNCH(128);
    else return hipErrorInvalidValue;
#undef C0_LAUNCH
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
    float eps, int *flag, OutClamp oc) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int nv = width >> 2;
    const f32x4 *xr = (const f32x4 *)(x + row * width);
    // Every operand of the row is loaded before any arithmetic or store (one
    // memory round trip); chunks past the width load its last chunk and take
    // no part.
    f32x4 v[NC], w1v[NC], rv[NC], w2v[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = min(lane + 64 * c, nv - 1);
        v[c] = xr[i];
        if (w1) w1v[c] = ((const f32x4 *)w1)[i];
        if (res) rv[c] = ((const f32x4 *)(res + row * width))[i];
        if (w2) w2v[c] = ((const f32x4 *)w2)[i];
    }
    bool ok = true;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (lane + 64 * c < nv && w1) {
            v[c] = clamp4(v[c], -c1, c1);
            ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
        }
    }
    if (w1) {
        ss = wave_sum(ss);
        const float inv = rms_inverse(ss, width, eps);
        ok = ok && isfinite(ss);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int i = lane + 64 * c;
            if (i < nv) v[c] = v[c] * inv * w1v[c];
        }
    }
    float ss2 = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i < nv) {
            if (res) v[c] = rv[c] + v[c] * rw;
            ok = ok && finite4(v[c]);
            if (h_out) {
                if (w2) {
                    ((f32x4 *)(h_out + row * width))[i] = v[c];
                } else {
                    for (int k = 0; k < oc.copies; ++k)
                        ((f32x4 *)(h_out + k * oc.stride + row * width))[i] =
                            clamp4(v[c], oc.lo[k], oc.hi[k]);
                }
            }
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
                const f32x4 y = v[c] * inv * w2v[c];
                ok = ok && finite4(y);
                for (int k = 0; k < oc.copies; ++k)
                    ((f32x4 *)(n_out + k * oc.stride + row * width))[i] = clamp4(y, oc.lo[k], oc.hi[k]);
            }
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_audio_rows(const float *x, float c1, const float *w1, const float *res, float rw,
                             float *h_out, float c2, const float *w2, float *n_out, int64_t rows,
                             int width, float eps, int *flag, hipStream_t s, const OutClamp &oc) {
    if (rows <= 0) return hipSuccess;
    if (width <= 0 || width % 4 || width > 2048 || oc.copies < 1 || oc.copies > 3)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4));
#define AR_LAUNCH(NC)                                                                        \
    hipLaunchKernelGGL(audio_rows_kernel<NC>, grid, dim3(256), 0, s, x, c1, w1, res, rw, h_out, \
                       c2, w2, n_out, rows, width, eps, flag, oc)
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
// One workgroup of AW waves per (block of `chunk` query rows of a clip,
// head): every query of a block shares the same `context` keys and values,
// so the workgroup stages them once in LDS (keys scaled by k_scale, key rows padded to an odd number of
// 16-byte chunks so lanes reading different rows at one column hit different
// banks), together with the head's relative-position keys and the block's
// queries (scaled by qf[d] = q_scale * softplus(per_dim_scale[d])). All
// global loads are issued up front; the rest runs out of LDS.
//
// Scores: lane (g, ci) = (lane / KL, lane % KL) takes context entry ci for
// queries g, g + G, g + 2G, ... of the sub-block (G = 64 / KL query groups,
// QPL queries per lane). Context entry ci is key block*chunk + ci - (left-1)
// of the clip; it is valid for query row il when the key is in the clip,
// unmasked, and 0 <= il - key < left - 1. The score is
// tanh((q.k + q.relk[ci - offset]) / cap) * cap, each dot summed over d in
// order, the relative term only when 0 <= ci - offset < positions; invalid
// entries score -1e9. Each query's softmax reduces over its KL lanes.
//
// Values: lane t holds head dims t, t + 64, ...; for each context entry in
// order, every query adds weight * v (keys outside the clip are skipped; a
// zero weight adds an exact zero, as the values are finite). A masked query
// row, or one with no valid key, gets zeros.
//
// AW waves share one workgroup and its staged keys, values and relative
// keys; wave w takes query sub-blocks w, w + AW, ... of QB queries each.
constexpr int AW = 2;

// Elements 4c .. 4c+3 of a row of `hd` floats, zero past the end.
__device__ __forceinline__ f32x4 load_row4(const float *row, int c, int hd, bool vec) {
    if (vec) return ((const f32x4 *)row)[c];
    f32x4 r = {0.f, 0.f, 0.f, 0.f};
    if (4 * c + 0 < hd) r.x = row[4 * c + 0];
    if (4 * c + 1 < hd) r.y = row[4 * c + 1];
    if (4 * c + 2 < hd) r.z = row[4 * c + 2];
    if (4 * c + 3 < hd) r.w = row[4 * c + 3];
    return r;
}

template <int KL, int QPL, int TD>
__global__ __launch_bounds__(64 * AW) void audio_attn_kernel(AudioAttnArgs p) {
    constexpr int G = 64 / KL, QB = QPL * G;
    extern __shared__ f32x4 lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int blk = (int)(blockIdx.x / (unsigned)p.heads);
    const int h = (int)blockIdx.x - blk * p.heads;
    const int64_t r0 = p.blocks[blk];
    const int il0 = p.pos[r0], len = p.rowlen[r0];
    const int64_t base = r0 - il0;
    const int nq = min(p.chunk, len - il0);
    const int hd = p.head_dim, hd4 = (hd + 3) >> 2, rs = hd4 | 1;
    const int max_past = p.left - 1, left_window = p.left - 1;
    const int kfirst = il0 - max_past;  // clip row of context entry 0
    f32x4 *ks = lds;
    f32x4 *rk = ks + p.context * rs;
    f32x4 *vs = rk + p.positions * rs;
    f32x4 *qs = vs + p.context * hd4 + wave * QB * hd4;
    // 16-byte loads when every row start is 16-byte aligned
    const bool vec = (hd & 3) == 0 && ((p.ldq | p.ldk | p.ldv) & 3) == 0 &&
                     (((uintptr_t)p.q | (uintptr_t)p.k | (uintptr_t)p.v | (uintptr_t)p.relk |
                       (uintptr_t)p.qf) & 15) == 0;

    // Staging issues SB loads per thread before any LDS store, so their
    // latencies overlap.
    constexpr int SB = 4, NT = 64 * AW;
    const int nkv = p.context * hd4;
    for (int i0 = threadIdx.x; i0 < nkv; i0 += SB * NT) {
        f32x4 kv[SB], vv[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            const int idx = i0 + u * NT;
            kv[u] = vv[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            const int ci = idx / hd4, c = idx - ci * hd4, kl = kfirst + ci;
            if (idx < nkv && kl >= 0 && kl < len) {
                kv[u] = load_row4(p.k + (base + kl) * p.ldk + (int64_t)h * hd, c, hd, vec);
                vv[u] = load_row4(p.v + (base + kl) * p.ldv + (int64_t)h * hd, c, hd, vec);
            }
        }
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            const int idx = i0 + u * NT;
            const int ci = idx / hd4, c = idx - ci * hd4;
            if (idx < nkv) {
                ks[ci * rs + c] = kv[u] * p.k_scale;
                vs[ci * hd4 + c] = vv[u];
            }
        }
    }
    const int nr = p.positions * hd4;
    for (int i0 = threadIdx.x; i0 < nr; i0 += SB * NT) {
        f32x4 rv[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            const int idx = i0 + u * NT;
            const int pi = idx / hd4, c = idx - pi * hd4;
            rv[u] = idx < nr ? load_row4(p.relk + ((int64_t)pi * p.heads + h) * hd, c, hd, vec)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < SB; ++u) {
            const int idx = i0 + u * NT;
            const int pi = idx / hd4, c = idx - pi * hd4;
            if (idx < nr) rk[pi * rs + c] = rv[u];
        }
    }
    // This wave's queries q0 .. q0 + nb - 1 (zeros for the rest of the sub-block).
    auto stage_queries = [&](int q0, int nb) {
        for (int i0 = lane; i0 < QB * hd4; i0 += SB * 64) {
            f32x4 qv[SB];
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                const int idx = i0 + u * 64;
                const int qi = idx / hd4, c = idx - qi * hd4;
                qv[u] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (idx < QB * hd4 && qi < nb)
                    qv[u] = load_row4(p.q + (r0 + q0 + qi) * p.ldq + (int64_t)h * hd, c, hd, vec) *
                            load_row4(p.qf, c, hd, vec);
            }
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                const int idx = i0 + u * 64;
                if (idx < QB * hd4) qs[idx] = qv[u];
            }
        }
    };

    const int ci = lane % KL, g = lane / KL;
    const int crow = min(ci, p.context - 1) * rs;
    const int kl = kfirst + ci;
    const bool key_ok = ci < p.context && kl >= 0 && kl < len && p.mask[base + kl];
    bool ok = true;
    stage_queries(wave * QB, min(QB, nq - wave * QB));
    // Every wave runs the same number of iterations (the barriers); a wave
    // past the block's last query has nb <= 0 and writes nothing.
    for (int qb0 = 0; qb0 < nq; qb0 += AW * QB) {
        const int q0 = qb0 + wave * QB;
        const int nb = min(QB, nq - q0);
        if (qb0 > 0) {
            __syncthreads();  // the previous sub-block's queries consumed
            stage_queries(q0, nb);
        }
        __syncthreads();
        int rrow[QPL];
        float sk[QPL], sr[QPL];
#pragma unroll
        for (int j = 0; j < QPL; ++j) {
            const int rel = ci - (q0 + g + G * j);
            rrow[j] = min(max(rel, 0), p.positions - 1) * rs;
            sk[j] = 0.f;
            sr[j] = 0.f;
        }
        for (int c = 0; c < hd4; ++c) {
            const f32x4 kv = ks[crow + c];
#pragma unroll
            for (int j = 0; j < QPL; ++j) {
                const f32x4 qv = qs[(g + G * j) * hd4 + c];
                const f32x4 rv = rk[rrow[j] + c];
                sk[j] += qv.x * kv.x;
                sk[j] += qv.y * kv.y;
                sk[j] += qv.z * kv.z;
                sk[j] += qv.w * kv.w;
                sr[j] += qv.x * rv.x;
                sr[j] += qv.y * rv.y;
                sr[j] += qv.z * rv.z;
                sr[j] += qv.w * rv.w;
            }
        }
        float wgt[QPL];
        bool live[QPL];
#pragma unroll
        for (int j = 0; j < QPL; ++j) {
            const int q = g + G * j;
            const int il = il0 + q0 + q;
            const int rel = ci - (q0 + q);
            const bool valid = q < nb && key_ok && il - kl >= 0 && il - kl < left_window;
            float score = -1.0e9f;
            if (valid) {
                const float dot = (rel >= 0 && rel < p.positions) ? sk[j] + sr[j] : sk[j];
                score = tanhf(dot / p.cap) * p.cap;
            }
            const float m = group_reduce<KL, true>(ci < p.context ? score : -INFINITY);
            const float e = ci < p.context ? expf(score - m) : 0.0f;
            const float sum = group_reduce<KL, false>(e);
            live[j] = q < nb && p.mask[r0 + q0 + q] && !(m <= -1.0e9f / 2.0f);
            if (live[j] && !(isfinite(sum) && sum > 0.0f)) ok = false;
            wgt[j] = e / sum;
        }
        float acc[QB][TD];
#pragma unroll
        for (int q = 0; q < QB; ++q)
#pragma unroll
            for (int t = 0; t < TD; ++t) acc[q][t] = 0.f;
        for (int c = 0; c < p.context; ++c) {
            const int kc = kfirst + c;
            if (kc < 0 || kc >= len) continue;
            const float *vr = (const float *)(vs + c * hd4);
            float vv[TD];
#pragma unroll
            for (int t = 0; t < TD; ++t) vv[t] = lane + 64 * t < hd ? vr[lane + 64 * t] : 0.f;
#pragma unroll
            for (int j = 0; j < QPL; ++j)
#pragma unroll
                for (int gg = 0; gg < G; ++gg) {
                    const int q = gg + G * j;
                    if (q >= nb) continue;
                    const float w = __int_as_float(
                        __builtin_amdgcn_readlane(__float_as_int(wgt[j]), c + KL * gg));
#pragma unroll
                    for (int t = 0; t < TD; ++t) acc[q][t] += w * vv[t];
                }
        }
#pragma unroll
        for (int j = 0; j < QPL; ++j)
#pragma unroll
            for (int gg = 0; gg < G; ++gg) {
                const int q = gg + G * j;
                if (q >= nb) continue;
                const bool on = __builtin_amdgcn_readlane((int)live[j], KL * gg) != 0;
                float *orow = p.out + (r0 + q0 + q) * p.ldo + (int64_t)h * hd;
#pragma unroll
                for (int t = 0; t < TD; ++t) {
                    const int d = lane + 64 * t;
                    if (d < hd) {
                        const float y = on ? acc[q][t] : 0.0f;
                        ok = ok && isfinite(y);
                        orow[d] = clamp_ref(y, p.out_lo, p.out_hi);
                    }
                }
            }
    }
    if (!ok) raise_flag(p.flag, FLAG_NONFINITE);
}

size_t audio_attention_lds(const AudioAttnArgs &a, int qb) {
    const int hd4 = (a.head_dim + 3) / 4, rs = hd4 | 1;
    return (size_t)((a.context + a.positions) * rs + (a.context + AW * qb) * hd4) * sizeof(f32x4);
}

template <int KL, int QPL, int TD>
hipError_t launch_audio_attn(const AudioAttnArgs &a, hipStream_t s) {
    const size_t lds = audio_attention_lds(a, QPL * (64 / KL));
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void *)audio_attn_kernel<KL, QPL, TD>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((audio_attn_kernel<KL, QPL, TD>), dim3((unsigned)(a.n_blocks * a.heads)),
                       dim3(64 * AW), lds, s, a);
    return hipGetLastError();
}

template <int KL, int TD>
hipError_t launch_audio_attn_q(const AudioAttnArgs &a, hipStream_t s) {
    // Queries per lane: enough for one block in one pass of the AW waves,
    // up to 8 (longer blocks take several passes).
    const int per = AW * (64 / KL);
    const int need = (a.chunk + per - 1) / per;
    if (need <= 1) return launch_audio_attn<KL, 1, TD>(a, s);
    if (need <= 2) return launch_audio_attn<KL, 2, TD>(a, s);
    if (need <= 3) return launch_audio_attn<KL, 3, TD>(a, s);
    if (need <= 4) return launch_audio_attn<KL, 4, TD>(a, s);
    return launch_audio_attn<KL, 8, TD>(a, s);
}

template <int KL>
hipError_t launch_audio_attn_d(const AudioAttnArgs &a, hipStream_t s) {
    switch ((a.head_dim + 63) / 64) {
        case 1: return launch_audio_attn_q<KL, 1>(a, s);
        case 2: return launch_audio_attn_q<KL, 2>(a, s);
        case 3: return launch_audio_attn_q<KL, 3>(a, s);
        default: return launch_audio_attn_q<KL, 4>(a, s);
    }
}

hipError_t launch_audio_attention(const AudioAttnArgs &a, hipStream_t s) {
    if (a.n_blocks <= 0) return hipSuccess;
    if (a.head_dim < 1 || a.head_dim > 256 || a.context < 1 || a.context > 64 || a.chunk < 1 ||
        a.positions < 1 || a.heads < 1 || a.n_blocks * a.heads > INT32_MAX)
        return hipErrorInvalidValue;
    return a.context <= 32 ? launch_audio_attn_d<32>(a, s) : launch_audio_attn_d<64>(a, s);
}

// ---- light convolution: causal depthwise conv + clamp + RMSNorm + SiLU -------
// One wave per row; taps ascend from row - (K - 1), rows before the clip's
// first row are skipped (audio.rs:1490-1503). dw is tap-major, [K, width].
template <int NC>
__global__ __launch_bounds__(256) void lconv_kernel(const float *__restrict__ gated,
                                                    const float *__restrict__ dw, int K,
                                                    const int32_t *__restrict__ pos, float clip,
                                                    const float *__restrict__ w, float *__restrict__ out,
                                                    int64_t rows, int width, float eps, int *flag,
                                                    float out_lo, float out_hi) {
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
                const f32x4 wt = ((const f32x4 *)(dw + (int64_t)tap * width))[i];
                acc.x += g.x * wt.x;
                acc.y += g.y * wt.y;
                acc.z += g.z * wt.z;
                acc.w += g.w * wt.w;
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
            ((f32x4 *)(out + row * width))[i] = clamp4(y, out_lo, out_hi);
        }
    }
    if (!ok) raise_flag(flag, FLAG_NONFINITE);
}

hipError_t launch_lconv(const float *gated, const float *dw, int K, const int32_t *pos, float clip,
                        const float *w, float *out, int64_t rows, int width, float eps, int *flag,
                        hipStream_t s, float out_lo, float out_hi) {
    if (rows <= 0) return hipSuccess;
    if (width % 4 || width > 2048) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4));
#define LC_LAUNCH(NC)                                                                           \
    hipLaunchKernelGGL(lconv_kernel<NC>, grid, dim3(256), 0, s, gated, dw, K, pos, clip, w, out, \
                       rows, width, eps, flag, out_lo, out_hi)
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
