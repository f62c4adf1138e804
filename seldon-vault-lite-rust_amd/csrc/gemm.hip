// FP32 GEMM on CDNA4 matrix cores: C = epilogue(A[M,K] . W[N,K]^T).
//
// This is the reference's `linear` (src/tensor/kernels.rs:577-685,
// out[r,c] = sum_k in[r,k] * w[c,k]) for every projection of the encoder:
// A is the packed activation matrix (all valid tokens of the batch, row
// major, K contiguous) and W the weight in the reference's [out, in] layout,
// so both operands are K-contiguous and no transpose is ever materialised.
//
// Design (gfx950):
//  * 256 threads = 4 wave64s in a 2x2 grid; each wave owns a (BM/2)x(BN/2)
//    block built from v_mfma_f32_32x32x2_f32 tiles (32 FMA/clk/SIMD, the FP32
//    matrix peak).
//  * K advances in BK = 32 slices staged through LDS, double buffered: the
//    next slice is fetched from HBM/L2 into registers while the MFMAs run
//    on the current one. Rows are padded to 36 floats so the 16 lanes of a
//    ds_read_b128 phase hit 64 distinct banks.
//  * Each lane reads float4 = 4 consecutive k of its row and feeds them to 4
//    MFMAs; lanes 0-31 carry k..k+3 and lanes 32-63 k+4..k+7 of the same 8-k
//    step, a k-permutation applied identically to A and W, so the sum over
//    k is unchanged.
//  * Tiles are numbered M-major with N fastest and remapped so consecutive
//    tiles land on the same XCD: the N tiles that share an A block hit that
//    XCD's L2 instead of HBM.
//  * Epilogues fuse the elementwise op that follows each projection in
//    text.rs (PLE scale, GeGLU, GELU-gate x per-layer input).
#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

template <int BM, int BN>
struct GemmShape {
    static constexpr int BK = 32;
    static constexpr int LDS = BK + 4;
    static constexpr int WM = BM / 2;
    static constexpr int WN = BN / 2;
    static constexpr int TM = WM / 32;
    static constexpr int TN = WN / 32;
    static constexpr int A_F4 = BM * BK / 4 / 256;
    static constexpr int W_F4 = BN * BK / 4 / 256;
};

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_nt_mfma(GemmArgs p, int tiles_m, int tiles_n) {
    using S = GemmShape<BM, BN>;
    __shared__ float As[2][BM * S::LDS];
    __shared__ float Ws[2][BN * S::LDS];

    // XCD-aware remap: hardware dispatches workgroup b to XCD b % 8.
    const int ntiles = tiles_m * tiles_n;
    const int bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3;
    const int q8 = ntiles >> 3, r8 = ntiles & 7;
    const int tile = xcd * q8 + min(xcd, r8) + local;
    const int tm = tile / tiles_n, tn = tile - tm * tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, hh = lane >> 5;
    const int M = p.M, N = p.N, K = p.K;

    f32x16 acc[S::TM][S::TN];
#pragma unroll
    for (int i = 0; i < S::TM; ++i)
#pragma unroll
        for (int j = 0; j < S::TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    f32x4 ra[S::A_F4], rw[S::W_F4];
    auto load_global = [&](int k0) {
#pragma unroll
        for (int i = 0; i < S::A_F4; ++i) {
            const int f = tid + 256 * i, row = f >> 3, gk = k0 + ((f & 7) << 2);
            const int gm = m0 + row;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (gm < M && gk < K) v = *(const f32x4 *)(p.A + (int64_t)gm * p.lda + gk);
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < S::W_F4; ++i) {
            const int f = tid + 256 * i, row = f >> 3, gk = k0 + ((f & 7) << 2);
            const int gn = n0 + row;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (gn < N && gk < K) v = *(const f32x4 *)(p.W + (int64_t)gn * p.ldw + gk);
            rw[i] = v;
        }
    };
    auto store_lds = [&](int buf) {
#pragma unroll
        for (int i = 0; i < S::A_F4; ++i) {
            const int f = tid + 256 * i;
            *(f32x4 *)&As[buf][(f >> 3) * S::LDS + ((f & 7) << 2)] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < S::W_F4; ++i) {
            const int f = tid + 256 * i;
            *(f32x4 *)&Ws[buf][(f >> 3) * S::LDS + ((f & 7) << 2)] = rw[i];
        }
    };

    const int nk = (K + S::BK - 1) / S::BK;
    load_global(0);
    store_lds(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_global((kt + 1) * S::BK);
        const float *as = &As[cur][(wm * S::WM + l32) * S::LDS + 4 * hh];
        const float *ws = &Ws[cur][(wn * S::WN + l32) * S::LDS + 4 * hh];
#pragma unroll
        for (int kk = 0; kk < S::BK; kk += 8) {
            f32x4 a[S::TM], b[S::TN];
#pragma unroll
            for (int i = 0; i < S::TM; ++i) a[i] = *(const f32x4 *)(as + i * 32 * S::LDS + kk);
#pragma unroll
            for (int j = 0; j < S::TN; ++j) b[j] = *(const f32x4 *)(ws + j * 32 * S::LDS + kk);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < S::TM; ++i)
#pragma unroll
                    for (int j = 0; j < S::TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s],
                                                                         acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_lds(cur ^ 1);
        __syncthreads();
    }

    // Epilogue. Accumulator register r of a 32x32 tile holds row
    // 8*(r/4) + 4*(lane/32) + r%4 and column lane%32.
    const int mw = m0 + wm * S::WM, nw = n0 + wn * S::WN;
#pragma unroll
    for (int i = 0; i < S::TM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = mw + i * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
            if (m >= M) continue;
            float *crow = p.C + (int64_t)m * p.ldc;
            if constexpr (EPI == EPI_GEGLU) {
#pragma unroll
                for (int j = 0; j < S::TN; j += 2) {
                    const int oc = nw / 2 + (j / 2) * 32 + l32;
                    if (oc < p.n_out) crow[oc] = gelu_tanh(acc[i][j][r]) * acc[i][j + 1][r];
                }
            } else {
#pragma unroll
                for (int j = 0; j < S::TN; ++j) {
                    const int n = nw + j * 32 + l32;
                    if (n >= N) continue;
                    float v = acc[i][j][r];
                    if constexpr (EPI == EPI_SCALE) v = v * p.alpha;
                    if constexpr (EPI == EPI_GELU_MUL)
                        v = gelu_tanh(v) * p.aux[(int64_t)m * p.ldaux + n];
                    crow[n] = v;
                }
            }
        }
    }
}

// One thread per output element; any K. Kept for shapes the MFMA kernel's
// float4 staging cannot take (K or a leading dimension not a multiple of 4).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_nt_simple(GemmArgs p) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int ncols = EPI == EPI_GEGLU ? p.n_out : p.N;
    if (idx >= (int64_t)p.M * ncols) return;
    const int m = (int)(idx / ncols), n = (int)(idx % ncols);
    const float *a = p.A + (int64_t)m * p.lda;
    float *crow = p.C + (int64_t)m * p.ldc;
    if constexpr (EPI == EPI_GEGLU) {
        // Interleaved rows: gate row of column n is 64*(n/32) + n%32, up row +32.
        const float *wg = p.W + (int64_t)(64 * (n / 32) + n % 32) * p.ldw;
        const float *wu = wg + 32 * p.ldw;
        float g = 0.f, u = 0.f;
        for (int k = 0; k < p.K; ++k) {
            g += a[k] * wg[k];
            u += a[k] * wu[k];
        }
        crow[n] = gelu_tanh(g) * u;
    } else {
        const float *w = p.W + (int64_t)n * p.ldw;
        float s = 0.f;
        for (int k = 0; k < p.K; ++k) s += a[k] * w[k];
        if constexpr (EPI == EPI_SCALE) s = s * p.alpha;
        if constexpr (EPI == EPI_GELU_MUL) s = gelu_tanh(s) * p.aux[(int64_t)m * p.ldaux + n];
        crow[n] = s;
    }
}

template <int BM, int BN, int EPI>
static hipError_t launch_mfma(const GemmArgs &a, hipStream_t s) {
    const int tm = (a.M + BM - 1) / BM, tn = (a.N + BN - 1) / BN;
    hipLaunchKernelGGL((gemm_nt_mfma<BM, BN, EPI>), dim3(tm * tn), dim3(256), 0, s, a, tm, tn);
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_simple(const GemmArgs &a, hipStream_t s) {
    const int ncols = EPI == EPI_GEGLU ? a.n_out : a.N;
    const int64_t n = (int64_t)a.M * ncols;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_nt_simple<EPI>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       a);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs &a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return hipSuccess;
    const bool vec_ok = (a.K % 4 == 0) && (a.lda % 4 == 0) && (a.ldw % 4 == 0) &&
                        ((uintptr_t)a.A % 16 == 0) && ((uintptr_t)a.W % 16 == 0);
    if (!vec_ok) return launch_gemm_simple(a, s);
    switch (a.epi) {
        case EPI_STORE: return launch_mfma<128, 128, EPI_STORE>(a, s);
        case EPI_SCALE: return launch_mfma<128, 128, EPI_SCALE>(a, s);
        case EPI_GEGLU: return launch_mfma<128, 128, EPI_GEGLU>(a, s);
        case EPI_GELU_MUL: return launch_mfma<128, 128, EPI_GELU_MUL>(a, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_simple(const GemmArgs &a, hipStream_t s) {
    switch (a.epi) {
        case EPI_STORE: return launch_simple<EPI_STORE>(a, s);
        case EPI_SCALE: return launch_simple<EPI_SCALE>(a, s);
        case EPI_GEGLU: return launch_simple<EPI_GEGLU>(a, s);
        case EPI_GELU_MUL: return launch_simple<EPI_GELU_MUL>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace svl
