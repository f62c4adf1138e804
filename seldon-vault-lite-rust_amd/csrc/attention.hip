// Bidirectional grouped-query attention (src/tensor/kernels.rs:1037-1135)
// over packed ragged rows: every row of the batch is an independent
// reference call, so keys never cross a row boundary, positions restart at 0
// per row, and the sliding window is the reference's symmetric inclusive
// |i - j| <= r.
//
// MFMA kernel (head_dim 64 / 128 / 256). All query heads that share a KV
// head are flattened into "query vectors" v = pos * G + g (G = heads per KV
// head), which is exactly their order in the [T, heads, hd] layout. A
// workgroup takes 32 * WAVES query vectors of one row and one KV head and
// streams that row's keys through LDS in tiles of 32, so one K/V tile feeds
// all G heads (the single shared KV head of EmbeddingGemma).
//  * S^T = K . Q^T with v_mfma_f32_32x32x2_f32: A = K tile from LDS, B = the
//    wave's 32 query vectors held in registers for the whole pass. In the
//    transposed score tile each lane owns one query column, so the running
//    max / sum of the online softmax and the rescale of the output are
//    lane-local (one cross-half shuffle per tile).
//  * O^T += V^T . P^T: the probabilities are consumed straight from the S^T
//    accumulator registers as the B operand (register r of lane l is key
//    8*(r/4) + 4*(l/32) + r%4, the k index that MFMA step r expects), and
//    the A operand reads V with output-row i mapped to head dims i*NT..+NT so
//    each lane loads NT contiguous floats.
//  * Tiles outside the sliding window of every query in the block are
//    skipped; padding keys beyond the row length are zero-filled and masked.
//
// Generic kernel (any head_dim): one wave per (token, head), the reference's
// own order of operations (score row, max-subtracted exp, divide by the sum,
// p-weighted value rows in key order).
#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

constexpr int ATTN_WAVES = 4;

template <int N>
__device__ __forceinline__ void load_n(const float *src, float (&dst)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const f32x4 v = *(const f32x4 *)(src + i);
            dst[i] = v.x;
            dst[i + 1] = v.y;
            dst[i + 2] = v.z;
            dst[i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

template <int HD, int WAVES>
__global__ __launch_bounds__(64 * WAVES, 1) void attn_mfma_kernel(AttnArgs p) {
    constexpr int KT = 32;        // keys per tile
    constexpr int KS = HD + 4;    // padded LDS row strides
    constexpr int VS = HD + 4;
    constexpr int NQ = HD / 8;    // float4 query fragments per lane
    constexpr int NT = HD / 32;   // output tiles (head dims per lane row)
    constexpr int NTHR = 64 * WAVES;
    __shared__ float Ks[KT * KS];
    __shared__ float Vs[KT * VS];

    const AttnTile tile = p.tiles[blockIdx.x];
    const int G = p.nh / p.nkv;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int nvec = tile.len * G;
    const int v = tile.qv0 + wave * 32 + l32;
    const bool vvalid = v < nvec;
    const int vq = vvalid ? v : nvec - 1;
    const int qpos = vq / G;
    const int qhead = tile.kvh * G + (vq - qpos * G);
    const float *qrow = p.q + (int64_t)(tile.tok0 + qpos) * p.ldq + qhead * HD;

    f32x4 qf[NQ];
#pragma unroll
    for (int c = 0; c < NQ; ++c) qf[c] = *(const f32x4 *)(qrow + 8 * c + 4 * hh);

    f32x16 o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    const int v_last = min(tile.qv0 + 32 * WAVES, nvec) - 1;
    const int p_lo = tile.qv0 / G, p_hi = v_last / G;
    int k_lo = 0, k_hi = tile.len - 1;
    if (p.window >= 0) {
        k_lo = max(0, p_lo - p.window);
        k_hi = min(tile.len - 1, p_hi + p.window);
    }
    const float *kbase = p.k + (int64_t)tile.tok0 * p.ldk + tile.kvh * HD;
    const float *vbase = p.v + (int64_t)tile.tok0 * p.ldv + tile.kvh * HD;

    for (int k0 = (k_lo / KT) * KT; k0 <= k_hi; k0 += KT) {
        __syncthreads();
        constexpr int F4R = HD / 4;
        for (int i = threadIdx.x; i < KT * F4R; i += NTHR) {
            const int r = i / F4R, c4 = i - r * F4R;
            const int key = k0 + r;
            f32x4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
            if (key < tile.len) {
                kv = *(const f32x4 *)(kbase + (int64_t)key * p.ldk + 4 * c4);
                vv = *(const f32x4 *)(vbase + (int64_t)key * p.ldv + 4 * c4);
            }
            *(f32x4 *)&Ks[r * KS + 4 * c4] = kv;
            *(f32x4 *)&Vs[r * VS + 4 * c4] = vv;
        }
        __syncthreads();

        f32x16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.f;
        const float *kp = &Ks[l32 * KS + 4 * hh];
#pragma unroll
        for (int c = 0; c < NQ; ++c) {
            const f32x4 a = *(const f32x4 *)(kp + 8 * c);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], qf[c][j], s, 0, 0, 0);
        }

        float pr[16];
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r >> 2) + 4 * hh + (r & 3);
            const bool ok = vvalid && key < tile.len &&
                            (p.window < 0 || abs(qpos - key) <= p.window);
            pr[r] = ok ? s[r] * p.scale : -INFINITY;
            tmax = fmaxf(tmax, pr[r]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pr[r] = pr[r] == -INFINITY ? 0.f : expf(pr[r] - m_new);
            psum += pr[r];
        }
        psum += __shfl_xor(psum, 32, 64);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t] = o[t] * alpha;

#pragma unroll
        for (int si = 0; si < 16; ++si) {
            const int key = 8 * (si >> 2) + 4 * hh + (si & 3);
            float va[NT];
            load_n<NT>(&Vs[key * VS + l32 * NT], va);
#pragma unroll
            for (int t = 0; t < NT; ++t)
                o[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[t], pr[si], o[t], 0, 0, 0);
        }
    }

    if (vvalid) {
        const float inv = 1.0f / l_run;
        float *orow = p.out + (int64_t)(tile.tok0 + qpos) * p.ldo + qhead * HD;
        bool ok = isfinite(inv);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = 8 * (r >> 2) + 4 * hh + (r & 3);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float y = o[t][r] * inv;
                ok = ok && isfinite(y);
                orow[i * NT + t] = y;
            }
        }
        if (!ok) raise_flag(p.flag, FLAG_NONFINITE);
    }
}

constexpr int ATTN_SIMPLE_MAX_KEYS = 8192;

__global__ __launch_bounds__(64) void attn_simple_kernel(AttnArgs p) {
    __shared__ float sc[ATTN_SIMPLE_MAX_KEYS];
    const int64_t idx = blockIdx.x;
    const int64_t t = idx / p.nh;
    const int h = (int)(idx - t * p.nh);
    const int lane = threadIdx.x;
    const int pos = p.pos[t], len = p.rowlen[t];
    const int64_t tok0 = t - pos;
    const int g = h / (p.nh / p.nkv);
    int lo = 0, hi = len - 1;
    if (p.window >= 0) {
        lo = max(0, pos - p.window);
        hi = min(len - 1, pos + p.window);
    }
    const int width = hi - lo + 1;
    const float *q = p.q + t * p.ldq + (int64_t)h * p.hd;
    bool ok = true;
    for (int j = lane; j < width; j += 64) {
        const float *k = p.k + (tok0 + lo + j) * p.ldk + (int64_t)g * p.hd;
        float d = 0.f;
        for (int e = 0; e < p.hd; ++e) d += q[e] * k[e];
        const float s = d * p.scale;
        ok = ok && isfinite(s);
        sc[j] = s;
    }
    float m = -INFINITY;
    for (int j = lane; j < width; j += 64) m = fmaxf(m, sc[j]);
    m = wave_max(m);
    float sum = 0.f;
    for (int j = lane; j < width; j += 64) {
        const float e = expf(sc[j] - m);
        sc[j] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float *out = p.out + t * p.ldo + (int64_t)h * p.hd;
    for (int d = lane; d < p.hd; d += 64) {
        float acc = 0.f;
        for (int j = 0; j < width; ++j) {
            const float pj = sc[j] / sum;
            if (pj == 0.f) continue;
            acc += pj * p.v[(tok0 + lo + j) * p.ldv + (int64_t)g * p.hd + d];
        }
        ok = ok && isfinite(acc);
        out[d] = acc;
    }
    if (!ok) raise_flag(p.flag, FLAG_NONFINITE);
}

int attn_block_vectors(int hd) {
    return (hd == 64 || hd == 128 || hd == 256) ? 32 * ATTN_WAVES : 0;
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
    if (a.tokens <= 0) return hipSuccess;
    const dim3 block(64 * ATTN_WAVES);
    switch (a.hd) {
        case 64:
            hipLaunchKernelGGL((attn_mfma_kernel<64, ATTN_WAVES>), dim3(a.n_tiles), block, 0, s, a);
            return hipGetLastError();
        case 128:
            hipLaunchKernelGGL((attn_mfma_kernel<128, ATTN_WAVES>), dim3(a.n_tiles), block, 0, s,
                               a);
            return hipGetLastError();
        case 256:
            hipLaunchKernelGGL((attn_mfma_kernel<256, ATTN_WAVES>), dim3(a.n_tiles), block, 0, s,
                               a);
            return hipGetLastError();
        default:
            if (!a.pos || !a.rowlen) return hipErrorInvalidValue;
            hipLaunchKernelGGL(attn_simple_kernel, dim3((unsigned)(a.tokens * a.nh)), dim3(64), 0,
                               s, a);
            return hipGetLastError();
    }
}

}  // namespace svl
