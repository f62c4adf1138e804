// FP32 GEMM on CDNA4 matrix cores: C = epilogue(A[M,K] . W[N,K]^T).
//
// This is the reference's `linear` (src/tensor/kernels.rs:577-685,
// out[r,c] = sum_k in[r,k] * w[c,k]) for every projection of the encoder:
// A is the packed activation matrix (all valid tokens of the batch, row
// major, K contiguous) and W the weight in the reference's [out, in] layout,
// so both operands are K-contiguous and no transpose is ever materialised.
//
// Design (gfx950):
//  * 256 threads = 4 wave64s; WMW waves along M and 4 / WMW along N (2 x 2
//    unless a tile is only 16 rows per wave); each wave owns a block of
//    v_mfma_f32_16x16x4_f32 tiles (16 FMA/clk/SIMD per instruction, the FP32
//    matrix peak). 16 x 16 output tiles keep one wave's dependent MFMA chain
//    at K / 4 instructions, so small-M launches (one short row) split the
//    output into many short chains instead of a few long ones.
//  * K advances in BK-wide slices that go straight from HBM/L2 into LDS with
//    buffer_load_dwordx4 ... lds (no register staging) through 2-4 LDS
//    stages: the DMAs of the next slices are in flight while the MFMAs
//    consume slice k, with one barrier per slice. Buffer resources bound
//    each operand to its valid rows, so the ragged M tail (and N tail) reads
//    zeros without branches.
//  * LDS rows are unpadded; 16-byte chunks are XOR-swizzled by row
//    (chunk ^ (row / 2 or 1) % chunks_per_row) on the way in, so the 16-row
//    fragment loads (one ds_read_b128 per lane) hit distinct banks.
//  * Lane l reads float4 = k0 + 4 (l / 16) .. + 3 of row l % 16 and feeds
//    element s to MFMA s, so MFMA s of a 16-k group sums k0 + s, k0 + 4 + s,
//    k0 + 8 + s, k0 + 12 + s; A and W use the same permutation, so the sum
//    over k is unchanged. Every output element sees the same MFMA sequence
//    over k whatever the tile shape, so results do not depend on the tile
//    chosen or on a row's position in the batch.
//  * The tile shape is chosen per launch from the grid's per-CU work:
//    128x128 (3 workgroups per CU) for large grids, 128x64 or 64x64 (4 per
//    CU) when bigger tiles would leave CUs idle or unevenly loaded, 32x32
//    when even 64x64 tiles would not cover the GPU once.
//  * Tiles are remapped so each XCD runs a contiguous range of the tile
//    list, N fastest (the N tiles that share an A block hit that XCD's L2);
//    launches of 128 M blocks or more with the whole GPU (32 or more when
//    the launch shares the GPU with other streams) order the range in
//    groups of 8 M blocks, M fastest within an N block and the N blocks of
//    every second group in reverse, so the tiles in flight on an XCD share a
//    few A blocks and W panels.
//  * Epilogues fuse the elementwise op that follows each projection in
//    text.rs (PLE scale, GeGLU, GELU-gate x per-layer input).
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

template <int BM, int BN>
struct GemmShape {
    static_assert(BM % 64 == 0 && BN % 64 == 0, "2x2 waves of 16x16 MFMA tiles");
    static constexpr int BK = 32;
    static constexpr int LDS = BK + 4;
    static constexpr int WM = BM / 2;
    static constexpr int WN = BN / 2;
    static constexpr int TM = WM / 16;
    static constexpr int TN = WN / 16;
    static constexpr int A_F4 = BM * BK / 4 / 256;
    static constexpr int W_F4 = BN * BK / 4 / 256;
};

// True for the epilogues whose W rows come in interleaved 32-row pairs.
template <int EPI>
constexpr bool paired_epi() {
    return EPI == EPI_GEGLU || EPI == EPI_CLIP_GLU;
}

template <int EPI>
constexpr bool clipped_epi() {
    return EPI == EPI_CLIP_STORE || EPI == EPI_CLIP_SILU || EPI == EPI_CLIP_GLU;
}

// Clip segment of an output tile starting at column n0 (tiles never straddle
// segments: the host keeps clip_cols a multiple of the widest tile).
__device__ __forceinline__ int clip_segment(const GemmArgs &p, int n0) {
    return p.clip_cols > 0 ? n0 / p.clip_cols : 0;
}

// Epilogue shared by the GEMM kernels. The MFMAs take the W fragment as
// their first operand, so a 16x16 accumulator tile is C transposed: lane l
// holds row l % 16 of the tile and its four consecutive columns
// 4 (l / 16) .. + 3, stored as one float4 (pairs of adjacent tiles are
// stored through store_pair). Paired epilogues take the 64-column groups of
// W (32 first-operand rows, then 32 second-operand rows): tiles j and j + 2
// of each group of four.
__device__ __forceinline__ void store_cols4(float *crow, int n0, int limit, bool vec,
                                            const f32x4 &v) {
    if (vec && n0 + 3 < limit) {
        *(f32x4 *)(crow + n0) = v;
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (n0 + r < limit) crow[n0 + r] = v[r];
    }
}

// Value lane l16 ^ 8 of the same 16-lane row holds (DPP row_ror:8).
__device__ __forceinline__ f32x4 row_swap8(f32x4 v) {
    f32x4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        r[c] = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[c]), 0x128, 0xF, 0xF, false));
    return r;
}

// Epilogue value of accumulator element r of 16x16 block (i, j) at row m,
// column n (unpaired epilogues).
template <int EPI>
__device__ __forceinline__ float epi_value(const GemmArgs &p, float x, int m, int n, float olo,
                                           float ohi) {
    if constexpr (EPI == EPI_SCALE) x = x * p.alpha;
    if constexpr (EPI == EPI_GELU_MUL)
        x = gelu_tanh(x) * (m < p.M && n < p.N ? p.aux[(int64_t)m * p.ldaux + n] : 0.f);
    if constexpr (EPI == EPI_BIAS) x = x + (n < p.N ? p.aux[n] : 0.f);
    if constexpr (EPI == EPI_CLIP_STORE) x = clamp_ref(x, olo, ohi);
    if constexpr (EPI == EPI_CLIP_SILU)
        x = clamp_ref(silu_ref(clamp_ref(x, olo, ohi)), p.post_lo, p.post_hi);
    return x;
}

// Stores a pair of horizontally adjacent 16x16 output blocks, X (columns
// cx .. cx + 15) and Y (cx + 16 .. cx + 31), rows r0 .. r0 + 15: lane l holds
// row r0 + l % 16, columns + 4 (l / 16) .. + 3 of each. Lanes with l % 16 < 8
// trade their Y values for the X values of lane l ^ 8, so each of the two
// stores writes 8 rows x 128 contiguous bytes (rows r0 .. r0 + 7, then
// r0 + 8 .. r0 + 15) instead of 16 rows x 64 bytes, and every 128-byte line
// of the output is written whole by one instruction.
__device__ __forceinline__ void store_pair(const GemmArgs &p, int limit, bool vec, int r0, int cx,
                                           int l16, int g, const f32x4 &X, const f32x4 &Y) {
    const bool lo = l16 < 8;
    const f32x4 t = row_swap8(lo ? Y : X);
    const int ra = r0 + (l16 & 7), col = (lo ? cx : cx + 16) + 4 * g;
    if (ra < p.M) store_cols4(p.C + (int64_t)ra * p.ldc, col, limit, vec, lo ? X : t);
    if (ra + 8 < p.M) store_cols4(p.C + (int64_t)(ra + 8) * p.ldc, col, limit, vec, lo ? t : Y);
}

// aux_pre (EPI_GELU_MUL, optional): the aux values of every accumulator
// element, loaded by the caller ahead of the K loop (aux_load below).
template <int TM, int TN, int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs &p, const f32x4 (&acc)[TM][TN],
                                              int mw, int nw, int l16, int g, int seg,
                                              const f32x4 (*aux_pre)[TN] = nullptr) {
    float olo = 0.f, ohi = 0.f;
    if constexpr (clipped_epi<EPI>()) {
        olo = p.clip[seg][2];
        ohi = p.clip[seg][3];
    }
    const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)p.C & 15) == 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = mw + i * 16 + l16;
        if constexpr (paired_epi<EPI>()) {
#pragma unroll
            for (int j = 0; j < TN; j += 4) {
                f32x4 v[2];
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float x = acc[i][j + u][r], y = acc[i][j + 2 + u][r];
                        if constexpr (EPI == EPI_GEGLU)
                            v[u][r] = gelu_tanh(x) * y;
                        else
                            v[u][r] = clamp_ref(x, olo, ohi) * sigmoid_ref(clamp_ref(y, olo, ohi));
                    }
                store_pair(p, p.n_out, vec, mw + i * 16, (nw + j * 16) / 2, l16, g, v[0], v[1]);
            }
        } else if constexpr (TN % 2 == 0) {
#pragma unroll
            for (int j = 0; j < TN; j += 2) {
                f32x4 v[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int n0 = nw + (j + u) * 16 + 4 * g;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if constexpr (EPI == EPI_GELU_MUL)
                            if (aux_pre) {
                                v[u][r] = gelu_tanh(acc[i][j + u][r]) * aux_pre[i][j + u][r];
                                continue;
                            }
                        v[u][r] = epi_value<EPI>(p, acc[i][j + u][r], m, n0 + r, olo, ohi);
                    }
                }
                store_pair(p, p.N, vec, mw + i * 16, nw + j * 16, l16, g, v[0], v[1]);
            }
        } else {
            if (m >= p.M) continue;
            float *crow = p.C + (int64_t)m * p.ldc;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n0 = nw + j * 16 + 4 * g;
                f32x4 v;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (EPI == EPI_GELU_MUL)
                        if (aux_pre) {
                            v[r] = gelu_tanh(acc[i][j][r]) * aux_pre[i][j][r];
                            continue;
                        }
                    v[r] = epi_value<EPI>(p, acc[i][j][r], m, n0 + r, olo, ohi);
                }
                store_cols4(crow, n0, p.N, vec, v);
            }
        }
    }
}

// EPI_GELU_MUL: the aux values of a wave's TM x TN accumulator blocks (row
// mw + 16 i + l16, columns nw + 16 j + 4 g .. + 3), one float4 per block
// where the row is 16-byte aligned, zero outside the output. Loaded before
// the K loop, so their latency hides behind it instead of following it.
template <int TM, int TN>
__device__ __forceinline__ void aux_load(const GemmArgs &p, int mw, int nw, int l16, int g,
                                         f32x4 (&out)[TM][TN]) {
    const bool vec = (p.ldaux & 3) == 0 && ((uintptr_t)p.aux & 15) == 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = mw + i * 16 + l16;
        const float *row = p.aux + (int64_t)(m < p.M ? m : 0) * p.ldaux;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = nw + j * 16 + 4 * g;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (m < p.M) {
                if (vec && n + 3 < p.N) {
                    v = *(const f32x4 *)(row + n);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < p.N) v[r] = row[n + r];
                }
            }
            out[i][j] = v;
        }
    }
}

// Paired epilogue over two waves (short grids): the wave holding the first
// halves x of a 32-column pair block (wn = 0) receives the second halves y
// from its partner through LDS (yv: block (i, u) of the partner at
// yv[(2 i + u) * 64 + lane]) and stores the 32 output columns of the pair.
// Same values as the one-wave paired epilogue above.
template <int TM, int EPI>
__device__ __forceinline__ void gemm_epilogue_pair_split(const GemmArgs &p,
                                                         const f32x4 (&acc)[TM][2],
                                                         const f32x4 *yv, int mw, int nw, int l16,
                                                         int g) {
    float olo = 0.f, ohi = 0.f;
    if constexpr (clipped_epi<EPI>()) {
        olo = p.clip[0][2];
        ohi = p.clip[0][3];
    }
    const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)p.C & 15) == 0;
    const int lane = l16 + 16 * g;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        f32x4 v[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const f32x4 y4 = yv[(2 * i + u) * 64 + lane];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = acc[i][u][r], y = y4[r];
                if constexpr (EPI == EPI_GEGLU)
                    v[u][r] = gelu_tanh(x) * y;
                else
                    v[u][r] = clamp_ref(x, olo, ohi) * sigmoid_ref(clamp_ref(y, olo, ohi));
            }
        }
        store_pair(p, p.n_out, vec, mw + i * 16, nw / 2, l16, g, v[0], v[1]);
    }
}

template <int BM, int BN, int EPI, int MINB = 2>
__global__ __launch_bounds__(256, MINB) void gemm_nt_mfma(GemmArgs p, int tiles_m, int tiles_n) {
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
    const int l16 = lane & 15, g = lane >> 4;
    const int M = p.M, N = p.N, K = p.K;
    const int seg = clip_segment(p, n0);
    const float *A = p.A + (int64_t)seg * p.a_seg;

    f32x4 acc[S::TM][S::TN];
#pragma unroll
    for (int i = 0; i < S::TM; ++i)
#pragma unroll
        for (int j = 0; j < S::TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    f32x4 ra[S::A_F4], rw[S::W_F4];
    auto load_global = [&](int k0) {
#pragma unroll
        for (int i = 0; i < S::A_F4; ++i) {
            const int f = tid + 256 * i, row = f >> 3, gk = k0 + ((f & 7) << 2);
            const int gm = m0 + row;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (gm < M && gk < K) v = *(const f32x4 *)(A + (int64_t)gm * p.lda + gk);
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
        const float *as = &As[cur][(wm * S::WM + l16) * S::LDS + 4 * g];
        const float *ws = &Ws[cur][(wn * S::WN + l16) * S::LDS + 4 * g];
#pragma unroll
        for (int kk = 0; kk < S::BK; kk += 16) {
            f32x4 a[S::TM], b[S::TN];
#pragma unroll
            for (int i = 0; i < S::TM; ++i) a[i] = *(const f32x4 *)(as + i * 16 * S::LDS + kk);
#pragma unroll
            for (int j = 0; j < S::TN; ++j) b[j] = *(const f32x4 *)(ws + j * 16 * S::LDS + kk);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < S::TM; ++i)
#pragma unroll
                    for (int j = 0; j < S::TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[j][s], a[i][s],
                                                                         acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_lds(cur ^ 1);
        __syncthreads();
    }

    gemm_epilogue<S::TM, S::TN, EPI>(p, acc, m0 + wm * S::WM, n0 + wn * S::WN, l16, g, seg);
}

// M blocks per rasterization group of the DMA kernel's tile order, and the
// fewest M blocks of a launch that takes the grouped order: 128 for a launch
// with the whole GPU (below that the 1 x 128-token forward went from 2.00 to
// 2.04 ms and the audio tower lost 1 % with it; the T2 launches kept their
// time and fetched 2.6x less), 32 for one that shares the GPU with other
// streams (the T2 row groups, about 98 M blocks each: 1695-1696 against
// 1680-1690 embeddings/s, and the image tower 29.31-29.37 against
// 29.48-29.64 ms; 16 and 64 measured the same as 32).
constexpr int RASTER_M = 8, RASTER_MIN_TILES_M = 128, RASTER_MIN_TILES_M_SHARED = 32;

// Direct-to-LDS variant; requires K % BK == 0 and 16-byte aligned rows. NS
// LDS stages: NS - 1 slices are in flight while one is consumed. WMW waves
// along M, 4 / WMW along N.
template <int BM, int BN, int BK, int EPI, int MINB, int NS, int WMW, bool CONV = false,
          bool RASTER = false>
__global__ __launch_bounds__(256, MINB) void gemm_nt_dma(GemmArgs p, int tiles_m, int tiles_n) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int WNW = 4 / WMW;                // waves along N
    constexpr int WTM = BM / WMW, WTN = BN / WNW;
    constexpr int TM = WTM / 16, TN = WTN / 16;  // 16x16 tiles per wave
    constexpr int CPR = BK / 4;                 // 16-byte chunks per row
    constexpr int RPK = 64 / CPR;               // rows per 1 KB DMA instruction
    // Swizzle: chunk ^ (row / RPL) % SWZ. Rows of 64 and 128 bytes (BK 16
    // and 32) change the XOR every second row, rows of 256 bytes or more
    // (BK >= 64) every row. SQ_LDS_BANK_CONFLICT reads zero for the fragment
    // loads of both; 64-byte rows changing it every fourth row conflicted on
    // half the LDS cycles (without a measurable cost to the kernel).
    constexpr int RPL = BK >= 64 ? 1 : 2;
    constexpr int SWZ = CPR < 16 ? CPR : 16;
    constexpr int A_CH = BM / RPK / 4;          // DMA instructions per wave per slice
    constexpr int W_CH = BN / RPK / 4;
    static_assert(WMW == 1 || WMW == 2 || WMW == 4, "wave layout");
    static_assert(BK % 16 == 0 && WTM % 16 == 0 && WTN % 16 == 0 && A_CH >= 1 && W_CH >= 1,
                  "tile shape");
    // paired epilogues: 64-column wave tiles (x and y halves in one wave), or
    // 64-column workgroup tiles whose two wave columns hold x and y
    constexpr bool PAIR_SPLIT = paired_epi<EPI>() && TN == 2;
    static_assert(!paired_epi<EPI>() || TN % 4 == 0 || (PAIR_SPLIT && WNW == 2),
                  "paired epilogues take 64-column wave or workgroup tiles");
    static_assert(!PAIR_SPLIT || WMW * TM * 2 * 64 * 4 <= BM * BK, "pair exchange fits stage 0");
    static_assert(NS >= 2 && NS <= 4 && (NS - 2) * (A_CH + W_CH) < 64, "pipeline depth");
    // One LDS object per stage, addressed with compile-time stage indices, so
    // the compiler can see that the DMA filling one stage never aliases the
    // fragment reads of another and need not drain the DMA before reading.
    __shared__ float As0[BM * BK], As1[BM * BK], As2[NS > 2 ? BM * BK : 4], As3[NS > 3 ? BM * BK : 4];
    __shared__ float Ws0[BN * BK], Ws1[BN * BK], Ws2[NS > 2 ? BN * BK : 4], Ws3[NS > 3 ? BN * BK : 4];
    auto stage_a = [&](auto st) -> float * {
        constexpr int i = decltype(st)::value;
        if constexpr (i == 0) return As0;
        else if constexpr (i == 1) return As1;
        else if constexpr (i == 2) return As2;
        else return As3;
    };
    auto stage_w = [&](auto st) -> float * {
        constexpr int i = decltype(st)::value;
        if constexpr (i == 0) return Ws0;
        else if constexpr (i == 1) return Ws1;
        else if constexpr (i == 2) return Ws2;
        else return Ws3;
    };

    const int ntiles = tiles_m * tiles_n;
    const int bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3;
    const int q8 = ntiles >> 3, r8 = ntiles & 7;
    const int tile = xcd * q8 + min(xcd, r8) + local;
    int tm, tn;
    if constexpr (RASTER) {
        // Within that range, groups of RASTER_M M blocks run N block by N
        // block, M fastest: the tiles in flight together on an XCD then share
        // a few W panels and A blocks in its L2 (the T2 gate/up launch fetched
        // 188 against 491 MiB with N fastest, at the same speed). Odd groups
        // run the N blocks in reverse, so a group starts on the W panels the
        // one before it ended on (the same launch fetched 187 against 217 MiB,
        // at the same speed).
        const int gsize = RASTER_M * tiles_n, grp = tile / gsize, first = grp * RASTER_M;
        const int gm = min(RASTER_M, tiles_m - first), in = tile - grp * gsize;
        tm = uniform(first + in % gm);
        tn = uniform(grp & 1 ? tiles_n - 1 - in / gm : in / gm);
    } else {
        tm = uniform(tile / tiles_n);
        tn = tile - tm * tiles_n;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    // The wave index through v_readfirstlane: the LDS destinations of the
    // DMA instructions (M0) then come from scalar registers, set by one
    // s_mov each, instead of a v_readfirstlane before every instruction of
    // every slice (T2 gate/up 479 -> 466 us, the 64x64 projections 5 %).
    // The one- or two-chain tiles that spread their DMA over the steps keep
    // it in a vector register: the audio tower's K = 4096 FFN down took 198
    // against 206 us that way, and its tower 15.17 against 15.40 ms.
    constexpr bool CHAIN_SPREAD = TM * TN <= 2 && MINB >= 2;
    const int tid = threadIdx.x, lane = tid & 63,
              wave = CHAIN_SPREAD ? tid >> 6 : uniform(tid >> 6);
    const int wm = wave / WNW, wn = wave % WNW;
    const int l16 = lane & 15, g = lane >> 4;
    const int M = p.M, N = p.N;
    const int seg = uniform(clip_segment(p, n0));

    // Operand windows: [valid rows of this tile] x lda floats; reads past
    // the last valid row return zero. (Implicit im2col: the whole layer-0
    // output, every lane's offset computed per tap.)
    const __amdgpu_buffer_rsrc_t ra = CONV
        ? __builtin_amdgcn_make_buffer_rsrc((void *)uniform(p.A), (short)0,
                                            uniform((int)(p.conv_a_floats * 4)), 0x00020000)
        : __builtin_amdgcn_make_buffer_rsrc(
              (void *)uniform(p.A + (int64_t)seg * p.a_seg + (int64_t)m0 * p.lda), (short)0,
              uniform((int)(min(BM, M - m0) * p.lda * 4)), 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void *)uniform(p.W + (int64_t)n0 * p.ldw), (short)0,
        uniform((int)(min(BN, N - n0) * p.ldw * 4)), 0x00020000);
    int a_off[A_CH], w_off[W_CH];
    // implicit im2col: per A row of this lane, the layer-0 float offset of
    // tap (0, 0) channel 0 and the valid kt (bits 0-2) and kf (bits 3-5)
    int a_taps[CONV ? A_CH : 1];
#pragma unroll
    for (int q = 0; q < A_CH; ++q) {
        const int row = (wave * A_CH + q) * RPK + lane / CPR;
        const int c = (lane % CPR) ^ ((row / RPL) % SWZ);
        if constexpr (CONV) {
            a_off[q] = 0;
            a_taps[q] = 0;
            const int m = m0 + row;
            if (m < M) {
                const int r = m / p.conv_f1, f = m - r * p.conv_f1;
                const int base = p.conv_rows[3 * r], t = p.conv_rows[3 * r + 1],
                          len = p.conv_rows[3 * r + 2];
                int bits = 0;
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    const int it = 2 * t + k - 1, iff = 2 * f + k - 1;
                    if (it >= 0 && it < len && p.conv_mask[base + it]) bits |= 1 << k;
                    if (iff >= 0 && iff < p.conv_f0) bits |= 8 << k;
                }
                a_off[q] = ((base + 2 * t - 1) * p.conv_f0 + 2 * f - 1) * p.conv_c0 + 4 * c;
                a_taps[q] = bits;
            }
        } else {
            a_off[q] = (row * (int)p.lda + 4 * c) * 4;
        }
    }
#pragma unroll
    for (int q = 0; q < W_CH; ++q) {
        const int row = (wave * W_CH + q) * RPK + lane / CPR;
        const int c = (lane % CPR) ^ ((row / RPL) % SWZ);
        w_off[q] = (row * (int)p.ldw + 4 * c) * 4;
    }
    // DMA instruction q of a slice: A for q < A_CH, else W (q - A_CH)
    auto issue_one = [&](auto st, int k0, int q) {
        float *as = stage_a(st);
        float *ws = stage_w(st);
        if (q < A_CH) {
            if constexpr (CONV) {
                const int tap = k0 / p.conv_c0, kt = tap / 3, kf = tap - 3 * kt;
                const int delta = (kt * p.conv_f0 + kf) * p.conv_c0 + (k0 - tap * p.conv_c0);
                const bool ok = (a_taps[q] >> kt & 1) && (a_taps[q] >> (3 + kf) & 1);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra, (__attribute__((address_space(3))) void *)&as[(wave * A_CH + q) * 256], 16,
                    ok ? (a_off[q] + delta) * 4 : 0x7FFFFFF0, 0, 0, 0);
            } else {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra, (__attribute__((address_space(3))) void *)&as[(wave * A_CH + q) * 256], 16,
                    a_off[q], k0 * 4, 0, 0);
            }
        } else {
            const int r = q - A_CH;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (__attribute__((address_space(3))) void *)&ws[(wave * W_CH + r) * 256], 16,
                w_off[r], k0 * 4, 0, 0);
        }
    };
    auto issue = [&](auto st, int k0) {
        float *as = stage_a(st);
        float *ws = stage_w(st);
        if constexpr (CONV) {
            // a K slice lies within one tap: k0 = tap * C0 + channel offset
            const int tap = k0 / p.conv_c0, kt = tap / 3, kf = tap - 3 * kt;
            const int delta = (kt * p.conv_f0 + kf) * p.conv_c0 + (k0 - tap * p.conv_c0);
#pragma unroll
            for (int q = 0; q < A_CH; ++q) {
                const bool ok = (a_taps[q] >> kt & 1) && (a_taps[q] >> (3 + kf) & 1);
                // a tap outside the clip, the mask or the frequencies reads
                // past the window, as zero
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra, (__attribute__((address_space(3))) void *)&as[(wave * A_CH + q) * 256], 16,
                    ok ? (a_off[q] + delta) * 4 : 0x7FFFFFF0, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int q = 0; q < A_CH; ++q)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra, (__attribute__((address_space(3))) void *)&as[(wave * A_CH + q) * 256], 16,
                    a_off[q], k0 * 4, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < W_CH; ++q)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (__attribute__((address_space(3))) void *)&ws[(wave * W_CH + q) * 256], 16,
                w_off[q], k0 * 4, 0, 0);
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // 16-row fragment blocks start at multiples of 16, so a row's swizzle
    // depends on l16 only
    const int sw = (l16 / RPL) % SWZ;
    const int nk = p.K / BK;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    // EPI_GELU_MUL: the per-layer inputs of this wave's outputs, ahead of the
    // K loop (loaded before the first DMA: the loop's vmcnt waits, which
    // count only the DMAs issued after them, then also cover these loads)
    f32x4 auxv[EPI == EPI_GELU_MUL ? TM : 1][EPI == EPI_GELU_MUL ? TN : 1];
    if constexpr (EPI == EPI_GELU_MUL) aux_load<TM, TN>(p, m0 + wm * WTM, n0 + wn * WTN, l16, g, auxv);
    if (0 < nk) issue(S0{}, 0);
    if constexpr (NS > 2) if (1 < nk) issue(S1{}, BK);
    if constexpr (NS > 3) if (2 < nk) issue(S2{}, 2 * BK);
    // slice kt lives in stage kt % NS; the loop below is unrolled NS times so
    // every stage index is a constant
    auto step = [&](int kt, auto st) {
        constexpr int cur = decltype(st)::value;
        // this wave's DMA of slice kt has landed: only the NS - 2 later
        // slices (A_CH + W_CH instructions each) may still be in flight
        if (kt + NS - 2 < nk) wait_vmcnt<(NS - 2) * (A_CH + W_CH)>();
        else wait_vmcnt<0>();
        __syncthreads();   // ... and every wave's; slice kt-1 is no longer read
        constexpr bool CHAIN = TM * TN <= 2;  // one or two accumulator chains per wave
        // several workgroups per CU: spread the next slice's DMA issue over
        // the MFMAs (below)
        constexpr bool SPREAD = MINB >= 2;
        using NEXT = std::integral_constant<int, (cur + NS - 1) % NS>;
        const bool refill = kt + NS - 1 < nk;
        if constexpr (!SPREAD)
            if (refill) issue(NEXT{}, (kt + NS - 1) * BK);
        const float *as = stage_a(st) + (wm * WTM + l16) * BK;
        const float *ws = stage_w(st) + (wn * WTN + l16) * BK;
        auto frags = [&](int kk, f32x4 (&a)[TM], f32x4 (&b)[TN]) {
            const int pos = ((kk >> 2) + g) ^ sw;
#pragma unroll
            for (int i = 0; i < TM; ++i) a[i] = *(const f32x4 *)(as + i * 16 * BK + 4 * pos);
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = *(const f32x4 *)(ws + j * 16 * BK + 4 * pos);
        };
        // the four MFMA rounds of a 16-k step; after(s) runs behind round s
        auto mfmas = [&](const f32x4 (&a)[TM], const f32x4 (&b)[TN], auto &&after) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(b[j][s], a[i][s],
                                                                         acc[i][j], 0, 0, 0);
                after(s);
            }
        };
        if constexpr (CHAIN) {
            // One or two accumulator chains per wave (the small and middle
            // grids): the fragments of step kk + 16 are read while step kk's
            // MFMAs run, so the LDS latency is not added to every step of the
            // dependent chain. With several workgroups per CU the next
            // slice's DMA instructions are also spread over the steps, each
            // issued behind an MFMA, rather than all issued before the first
            // (each takes tens of cycles to issue, and the wave issues in
            // order): 3 % on 64x32 tiles. With one workgroup per CU (the
            // 32x32 and 32x64 tiles of a few short rows) that took 6.7 to
            // 7.8 us at 128 x 768 x 768, so there the slice is issued first.
            constexpr int NDMA = A_CH + W_CH, NSTEP = BK / 16;
            f32x4 a[TM], b[TN];
            frags(0, a, b);
#pragma unroll
            for (int kk = 0; kk < BK; kk += 16) {
                f32x4 na[TM], nb[TN];
                if (kk + 16 < BK) frags(kk + 16, na, nb);
                __builtin_amdgcn_sched_barrier(0);
                const int t = kk / 16;
                mfmas(a, b, [&](int s) {
                    if (s != 0) return;
                    if (SPREAD && refill) {
#pragma unroll
                        for (int q = 0; q < NDMA; ++q)
                            if (q * NSTEP / NDMA == t) issue_one(NEXT{}, (kt + NS - 1) * BK, q);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                });
                if (kk + 16 < BK) {
#pragma unroll
                    for (int i = 0; i < TM; ++i) a[i] = na[i];
#pragma unroll
                    for (int j = 0; j < TN; ++j) b[j] = nb[j];
                }
            }
        } else {
            // Larger wave tiles: with several workgroups per CU, DMA
            // instruction q of the next slice goes behind MFMA round
            // q * NR / NDMA of the first half of this slice's rounds rather
            // than all of them before its first MFMA (the T2 gate/up 467 ->
            // 462 us, the 128x128 projections of 18688 rows 495 -> 486 us;
            // over all the rounds, the last DMA issued at the slice's end,
            // 464 and 488 us, and the audio tower's FFN up 187 against 182 us).
            constexpr int NDMA = A_CH + W_CH, NR = BK / 16 * 2;  // MFMA rounds per half slice
#pragma unroll
            for (int kk = 0; kk < BK; kk += 16) {
                f32x4 a[TM], b[TN];
                frags(kk, a, b);
                const int r0 = kk / 16 * 4;
                mfmas(a, b, [&](int s) {
                    if constexpr (SPREAD) {
                        if (refill) {
#pragma unroll
                            for (int q = 0; q < NDMA; ++q)
                                if (q * NR / NDMA == r0 + s) issue_one(NEXT{}, (kt + NS - 1) * BK, q);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                });
            }
        }
    };
    for (int kt = 0; kt < nk; kt += NS) {
        step(kt, S0{});
        if (kt + 1 < nk) step(kt + 1, S1{});
        if constexpr (NS > 2) if (kt + 2 < nk) step(kt + 2, S2{});
        if constexpr (NS > 3) if (kt + 3 < nk) step(kt + 3, S3{});
    }
    if constexpr (PAIR_SPLIT) {
        __syncthreads();  // every wave is done reading the stages
        f32x4 *xch = (f32x4 *)As0 + wm * TM * 2 * 64;
        if (wn == 1) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int u = 0; u < 2; ++u) xch[(2 * i + u) * 64 + lane] = acc[i][u];
        }
        __syncthreads();
        if (wn == 0) gemm_epilogue_pair_split<TM, EPI>(p, acc, xch, m0 + wm * WTM, n0, l16, g);
    } else if constexpr (EPI == EPI_GELU_MUL) {
        gemm_epilogue<TM, TN, EPI>(p, acc, m0 + wm * WTM, n0 + wn * WTN, l16, g, seg, auxv);
    } else {
        gemm_epilogue<TM, TN, EPI>(p, acc, m0 + wm * WTM, n0 + wn * WTN, l16, g, seg);
    }
#endif
}

// One thread per output element; any K. Kept for shapes the MFMA kernel's
// float4 staging cannot take (K or a leading dimension not a multiple of 4).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_nt_simple(GemmArgs p) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int ncols = paired_epi<EPI>() ? p.n_out : p.N;
    if (idx >= (int64_t)p.M * ncols) return;
    const int m = (int)(idx / ncols), n = (int)(idx % ncols);
    const int seg = clipped_epi<EPI>() && p.clip_cols > 0 ? (paired_epi<EPI>() ? 0 : n / p.clip_cols) : 0;
    const float *a = p.A + (int64_t)seg * p.a_seg + (int64_t)m * p.lda;
    float *crow = p.C + (int64_t)m * p.ldc;
    float alo = 0.f, ahi = 0.f, olo = 0.f, ohi = 0.f;
    if constexpr (clipped_epi<EPI>()) {
        alo = p.clip[seg][0];
        ahi = p.clip[seg][1];
        olo = p.clip[seg][2];
        ohi = p.clip[seg][3];
    }
    if constexpr (paired_epi<EPI>()) {
        // Interleaved rows: first row of column n is 64*(n/32) + n%32, second +32.
        const float *wg = p.W + (int64_t)(64 * (n / 32) + n % 32) * p.ldw;
        const float *wu = wg + 32 * p.ldw;
        float g = 0.f, u = 0.f;
        for (int k = 0; k < p.K; ++k) {
            float x = a[k];
            if constexpr (clipped_epi<EPI>()) x = clamp_ref(x, alo, ahi);
            g += x * wg[k];
            u += x * wu[k];
        }
        if constexpr (EPI == EPI_GEGLU)
            crow[n] = gelu_tanh(g) * u;
        else
            crow[n] = clamp_ref(g, olo, ohi) * sigmoid_ref(clamp_ref(u, olo, ohi));
    } else {
        const float *w = p.W + (int64_t)n * p.ldw;
        float s = 0.f;
        for (int k = 0; k < p.K; ++k) {
            float x = a[k];
            if constexpr (clipped_epi<EPI>()) x = clamp_ref(x, alo, ahi);
            s += x * w[k];
        }
        if constexpr (EPI == EPI_SCALE) s = s * p.alpha;
        if constexpr (EPI == EPI_GELU_MUL) s = gelu_tanh(s) * p.aux[(int64_t)m * p.ldaux + n];
        if constexpr (EPI == EPI_BIAS) s = s + p.aux[n];
        if constexpr (EPI == EPI_CLIP_STORE) s = clamp_ref(s, olo, ohi);
        if constexpr (EPI == EPI_CLIP_SILU)
            s = clamp_ref(silu_ref(clamp_ref(s, olo, ohi)), p.post_lo, p.post_hi);
        crow[n] = s;
    }
}

template <int BM, int BN, int BK, int EPI, int MINB, int NS, int WMW = 2, bool CONV = false>
static hipError_t launch_dma(const GemmArgs &a, hipStream_t s) {
    const int tm = (a.M + BM - 1) / BM, tn = (a.N + BN - 1) / BN;
    if constexpr (!CONV) {
        if (tm >= (a.cus > 0 ? RASTER_MIN_TILES_M_SHARED : RASTER_MIN_TILES_M)) {
            hipLaunchKernelGGL((gemm_nt_dma<BM, BN, BK, EPI, MINB, NS, WMW, false, true>),
                               dim3(tm * tn), dim3(256), 0, s, a, tm, tn);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemm_nt_dma<BM, BN, BK, EPI, MINB, NS, WMW, CONV>), dim3(tm * tn),
                       dim3(256), 0, s, a, tm, tn);
    return hipGetLastError();
}

// Tile choice.
//  * A launch with the whole GPU: workgroups are spread round-robin over the
//    256 CUs, so it takes about ceil(tiles / 256) tile-times on its busiest
//    CU; the cost of a tile shape is that count times the tile's MAC count
//    over the shape's measured efficiency (128x128 at 3 per CU and 64x64 at
//    4 per CU: 1.0; 128x64 at 4 per CU: 0.95; 64x32 at 4 per CU: 0.93),
//    ties going to the larger tile (the audio tower's M = 3000 x 4096
//    projection: 250 us at 128x128, 275 us at 64x64). With 16x16 fragments
//    64x64 tiles keep up with larger ones (the 18688-token O projection:
//    168 us against 202 us for 128x64 tiles), and their finer grid wastes
//    less of the last round.
//  * A launch that shares the GPU with other streams (a.cus > 0, the text
//    path's row groups): 64x64 (O and down per group: 65 and 93 us against
//    75 and 110 us for 128x64); the other streams' work fills the partial
//    rounds that the cost model above optimises for.
//  * Grids that 64x64 tiles would not cover once (one short row, 128 tokens:
//    QKV at 6.9 us against 15.9 us for 64x64 tiles): 32x32 tiles, one 16x16
//    block per wave; paired epilogues 32x64 tiles whose two wave columns
//    hold the x and y halves of the pair block (two 16x16 blocks per wave),
//    joined through LDS for the epilogue.
//  * Otherwise paired epilogues keep the 32 + 32 columns of a pair in one
//    wave: 64x128 tiles (4 per CU; the 18688-token gate/up: 481 us against
//    502 us for 128x128), for the row groups too, with deeper pipelines below
//    two rounds of 128x128 tiles.
//  * Outputs of at most 32 columns (the audio subsampling's 32 channels):
//    128x32 tiles, the four waves stacked along M, instead of 64x64 tiles
//    that would spend half their MFMAs on zero columns.
//  * Stages: grids of at least two workgroups per CU keep two stages (their
//    co-resident workgroups hide each other's DMA latency, and a deeper
//    pipeline measured slower there); short grids, whose few workgroups run
//    the K loop alone, take as many stages as the LDS budget allows.
//    Grids that do not fill the GPU once (fewer tiles than CUs) also take
//    64-wide K slices, so each barrier is amortised over four times more
//    MFMAs (the k order, set by the 16-k groups, is the same for any slice
//    width).
template <int BM, int BN, int BK, int EPI, int MINB, int NS_DEEP>
static hipError_t launch_dma_staged(const GemmArgs &a, hipStream_t s) {
    // workgroups per CU that the deep pipeline's LDS allows (160 KB per CU)
    constexpr int FIT = 160 * 1024 / (NS_DEEP * (BM + BN) * BK * 4);
    constexpr int MINB_DEEP = FIT < MINB ? FIT : MINB;
    const int64_t t = (int64_t)((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    if constexpr (BM * BN <= 64 * 128)
        if (t < 256 && a.K % 64 == 0) return launch_dma<BM, BN, 64, EPI, 1, 3>(a, s);
    if (t < 2 * 256) return launch_dma<BM, BN, BK, EPI, MINB_DEEP, NS_DEEP>(a, s);
    return launch_dma<BM, BN, BK, EPI, MINB, 2>(a, s);
}

template <int EPI>
static hipError_t launch_dma_auto(const GemmArgs &a, hipStream_t s) {
    auto tiles = [&](int bm, int bn) {
        return (int64_t)((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn);
    };
    // Grids that 64x64 tiles would not cover once (a few short rows): the
    // smallest tiles, one 16x16 block per wave (paired: two, the x or the y
    // half of the pair), so each wave's MFMA chain is K / 4 (2 x K / 4)
    // instructions long.
    const bool tiny = tiles(64, 64) < 256 && a.K % 32 == 0;
    if constexpr (paired_epi<EPI>()) {
        if (tiny && tiles(32, 64) <= 256) {
            // 32x64 tiles: the x and y halves of each pair on two waves, so a
            // wave's chain is 2 x K / 4 MFMAs (gate/up at 128 tokens: 12.1 us
            // against 17.6 us for 64x64 tiles with one 16x64 block per wave;
            // three or four stages measured no faster). They fill the GPU
            // once at one workgroup per CU; larger grids take the rules below
            // (gate/up at 256 tokens 17.2 against 20.0 us).
            if (a.K % 128 == 0) return launch_dma<32, 64, 128, EPI, 1, 2, 2>(a, s);
            if (a.K % 64 == 0) return launch_dma<32, 64, 64, EPI, 1, 3, 2>(a, s);
            return launch_dma<32, 64, 32, EPI, 1, 4, 2>(a, s);
        }
        // concurrent row groups: 64x128x16 tiles at four per CU, as for the
        // whole batch (the T2 step 37.57-37.64 against 37.98-38.04 ms with
        // 128x128x16 tiles at three per CU, which had led before the DMA
        // issue moved behind the MFMAs; same box)
        if (a.cus > 0 && a.K % 16 == 0) return launch_dma<64, 128, 16, EPI, 4, 2>(a, s);
        if (tiles(128, 128) < 2 * 256) {
            // grids of a few thousand rows: tiles small enough to spread over
            // every CU (gate/up at 1040 / 2000 / 3016 rows: 34.7 / 63.8 / 88.0
            // us against 53.9 / 76.6 / 104.2 us for 64x128 tiles)
            if (a.K % 32 == 0) {
                if (tiles(64, 64) < 1280) return launch_dma<32, 64, 32, EPI, 4, 2, 2>(a, s);
                return launch_dma<64, 64, 32, EPI, 4, 2, 4>(a, s);
            }
            return launch_dma<64, 128, 16, EPI, 3, 4>(a, s);
        }
        return launch_dma<64, 128, 16, EPI, 4, 2>(a, s);
    } else {
        if (tiny) {
            // Wide K slices: fewer DMA round trips and barriers on a chain
            // that is mostly memory latency. 256-wide slices (two 64 KB
            // stages) took the 1 x 128-token forward from 1.837 to 1.811 ms
            // against 128-wide ones; 128-wide took O at 128 tokens from 7.6
            // to 7.0 us against 64-wide. Those hold one workgroup per CU, so
            // they serve grids of one round; larger ones take 64-wide slices
            // in three stages, three workgroups per CU (at 1040 tokens the
            // N = 768 projections 15.7 against 20.8 us, the PLE gate 9.1
            // against 11.3 us; at 520 tokens QKV 12.8 against 16.7 us).
            if (tiles(32, 32) <= 256) {
                if (a.K % 256 == 0) return launch_dma<32, 32, 256, EPI, 1, 2>(a, s);
                if (a.K % 128 == 0) return launch_dma<32, 32, 128, EPI, 1, 2>(a, s);
            }
            if (a.K % 64 == 0) return launch_dma<32, 32, 64, EPI, 1, 3>(a, s);
            return launch_dma<32, 32, 32, EPI, 1, 4>(a, s);
        }
        // The PLE gate (N = 256, K = 768, GELU x per-layer input): 64x32 tiles
        // at six per CU, whole batch or row group (T2 whole batch 68 against
        // 76 us for 64x64 tiles; three row groups together 62 against 66-73 us)
        if constexpr (EPI == EPI_GELU_MUL)
            if (a.K % 32 == 0) return launch_dma<64, 32, 32, EPI, 6, 2, 2>(a, s);
        if (a.cus > 0) {
            if (a.K % 32 == 0) return launch_dma<64, 64, 32, EPI, 4, 2>(a, s);
            if (tiles(128, 128) < 4 * 256) return launch_dma_staged<128, 64, 16, EPI, 4, 3>(a, s);
            return launch_dma_staged<128, 128, 16, EPI, 3, 3>(a, s);
        }
        if (a.N <= 32 && a.K % 32 == 0) return launch_dma<128, 32, 32, EPI, 4, 2, 4>(a, s);
        // The least work on the busiest CU, over the shape's efficiency. 64x32
        // tiles (one or two accumulator blocks per wave) run at 0.93 of 64x64
        // ones, and their finer grid evens out grids of a few thousand rows: at
        // 3000 rows N = 768 (K = 1536) took 63.7 against 70.9 us for 64x64
        // tiles (564 of them leave CUs with two or three) and N = 1536 74.6
        // against 79.4 us, while N = 1024 (752 64x64 tiles, three per CU)
        // took 190.6 against 205.8 us at K = 4096 on 64x64 tiles.
        auto per_cu = [&](int bm, int bn) { return (double)((tiles(bm, bn) + 255) / 256); };
        // 128x128 tiles run three at a time per CU, and a CU's last round
        // holds its remainder: their count is rounded up to whole rounds (the
        // 16384-row QKV, five per CU: 268 us against 230 us for 64x64 tiles;
        // the 3016-row QKV, one per CU: 52.6 against 49.0 us)
        const double c128 = std::ceil(per_cu(128, 128) / 3.0) * 3.0 * (128.0 * 128.0);
        const double c12864 = per_cu(128, 64) * (128.0 * 64.0) / 0.95;
        const double c64 = per_cu(64, 64) * (64.0 * 64.0);
        const double c6432 = a.K % 32 == 0 ? per_cu(64, 32) * (64.0 * 32.0) / 0.93 : 1e300;
        if (c6432 < c64 && c6432 < c128 && c6432 < c12864) return launch_dma<64, 32, 32, EPI, 4, 2, 2>(a, s);
        if (c64 < c128 && c64 < c12864) {
            if (a.K % 32 == 0) return launch_dma_staged<64, 64, 32, EPI, 4, 3>(a, s);
            return launch_dma_staged<64, 64, 16, EPI, 4, 4>(a, s);
        }
        if (c12864 < c128) return launch_dma_staged<128, 64, 16, EPI, 4, 3>(a, s);
        return launch_dma_staged<128, 128, 16, EPI, 3, 3>(a, s);
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
    const int ncols = paired_epi<EPI>() ? a.n_out : a.N;
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
    // Buffer offsets are 32-bit: an operand window must stay below 2 GiB.
    const bool dma_ok = a.K % 16 == 0 && (int64_t)128 * std::max(a.lda, a.ldw) * 4 < INT32_MAX;
    if (dma_ok) {
        switch (a.epi) {
            case EPI_STORE: return launch_dma_auto<EPI_STORE>(a, s);
            case EPI_SCALE: return launch_dma_auto<EPI_SCALE>(a, s);
            case EPI_GEGLU: return launch_dma_auto<EPI_GEGLU>(a, s);
            case EPI_GELU_MUL: return launch_dma_auto<EPI_GELU_MUL>(a, s);
            case EPI_BIAS: return launch_dma_auto<EPI_BIAS>(a, s);
            case EPI_CLIP_STORE: return launch_dma_auto<EPI_CLIP_STORE>(a, s);
            case EPI_CLIP_SILU: return launch_dma_auto<EPI_CLIP_SILU>(a, s);
            case EPI_CLIP_GLU: return launch_dma_auto<EPI_CLIP_GLU>(a, s);
        }
        return hipErrorInvalidValue;
    }
    switch (a.epi) {
        case EPI_STORE: return launch_mfma<128, 128, EPI_STORE>(a, s);
        case EPI_SCALE: return launch_mfma<128, 128, EPI_SCALE>(a, s);
        case EPI_GEGLU: return launch_mfma<128, 128, EPI_GEGLU>(a, s);
        case EPI_GELU_MUL: return launch_mfma<128, 128, EPI_GELU_MUL>(a, s);
        case EPI_BIAS: return launch_mfma<128, 128, EPI_BIAS>(a, s);
        case EPI_CLIP_STORE: return launch_mfma<128, 128, EPI_CLIP_STORE>(a, s);
        case EPI_CLIP_SILU: return launch_mfma<128, 128, EPI_CLIP_SILU>(a, s);
        case EPI_CLIP_GLU: return launch_mfma<128, 128, EPI_CLIP_GLU>(a, s);
    }
    return hipErrorInvalidValue;
}

// The implicit-im2col convolution: 128x32 tiles (the layer-1 GEMM has 8 to
// 32 output channels) or 64x64, 32-wide K slices that each lie within one
// tap. No column matrix is written: each lane's DMA reads its 16 bytes of the
// layer-0 output at the tap's offset, and taps outside the input read the
// zeros past the buffer window.
bool gemm_conv_ok(const GemmArgs &a) {
    return a.epi == EPI_STORE && a.conv_rows && a.conv_mask && a.conv_c0 > 0 &&
           a.conv_c0 % 32 == 0 && a.K == 9 * a.conv_c0 && a.conv_f0 > 0 && a.conv_f1 > 0 &&
           a.conv_a_floats > 0 && a.conv_a_floats * 4 < 0x7FFFFFF0 && a.ldw % 4 == 0 &&
           (uintptr_t)a.A % 16 == 0 && (uintptr_t)a.W % 16 == 0 &&
           (int64_t)128 * a.ldw * 4 < INT32_MAX;
}

hipError_t launch_gemm_conv(const GemmArgs &a, hipStream_t s) {
    if (a.M <= 0 || a.N <= 0) return hipSuccess;
    if (!gemm_conv_ok(a)) return hipErrorInvalidValue;
    if (a.N <= 32) return launch_dma<128, 32, 32, EPI_STORE, 4, 2, 4, true>(a, s);
    return launch_dma<64, 64, 32, EPI_STORE, 4, 2, 2, true>(a, s);
}

hipError_t launch_gemm_simple(const GemmArgs &a, hipStream_t s) {
    switch (a.epi) {
        case EPI_STORE: return launch_simple<EPI_STORE>(a, s);
        case EPI_SCALE: return launch_simple<EPI_SCALE>(a, s);
        case EPI_GEGLU: return launch_simple<EPI_GEGLU>(a, s);
        case EPI_GELU_MUL: return launch_simple<EPI_GELU_MUL>(a, s);
        case EPI_BIAS: return launch_simple<EPI_BIAS>(a, s);
        case EPI_CLIP_STORE: return launch_simple<EPI_CLIP_STORE>(a, s);
        case EPI_CLIP_SILU: return launch_simple<EPI_CLIP_SILU>(a, s);
        case EPI_CLIP_GLU: return launch_simple<EPI_CLIP_GLU>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace svl
