// Bidirectional grouped-query attention (src/tensor/kernels.rs:1037-1135)
// over packed ragged rows: every row of the batch is an independent
// reference call, so keys never cross a row boundary, positions restart at 0
// per row, and the sliding window is the reference's symmetric inclusive
// |i - j| <= r.
//
// MFMA kernels (head_dim 64 / 128 / 256). All query heads that share a KV
// head are flattened into "query vectors" v = pos * G + g (G = heads per KV
// head), which is exactly their order in the [T, heads, hd] layout. A work
// item is 128 query vectors of one row and one KV head; that row's keys
// stream through LDS in tiles, so one K/V tile feeds all G heads (the single
// shared KV head of EmbeddingGemma).
//  * attn16_kernel (below): K/V tiles by DMA, v_mfma_f32_16x16x4_f32
//    fragments, 16 vectors per wave. It runs every launch whose rows fit
//    32-bit buffer offsets (every row the models accept).
//  * attn_mfma_kernel: the register-staged fallback for longer rows, on
//    v_mfma_f32_32x32x2_f32 with 32 vectors per wave. S^T = K . Q^T with the
//    queries in registers; each lane owns one query column of the score
//    tile, so the online softmax is lane-local (one cross-half shuffle per
//    tile). O^T += V^T . P^T takes P straight from the score accumulators
//    (register r of lane l is key 8*(r/4) + 4*(l/32) + r%4, the k index MFMA
//    step r expects); V is read with output-row i mapped to head dims
//    i*NT..+NT so each lane loads NT contiguous floats.
//  * Tiles outside the sliding window of every query in the block are
//    skipped; padding keys beyond the row length are zero-filled and masked.
//
// Generic kernel (any head_dim): one wave per (token, head), the reference's
// own order of operations (score row, max-subtracted exp, divide by the sum,
// p-weighted value rows in key order).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

constexpr int ATTN_WAVES = 4;
constexpr float RESCALE_LOG2 = 8.0f;

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

// DMA kernel for head_dim 64, 128 and 256 on v_mfma_f32_16x16x4_f32
// fragments: each wave owns 16 query vectors, so its Q fragments and O^T
// accumulators take HD / 4 + HD / 4 registers (64 + 64 at head_dim 256).
// Keys stream in tiles of KT keys (16 at head_dim 256, 32 at 128 and 64:
// more MFMAs per barrier and softmax at the smaller head dims), so two or
// more workgroups of four waves
// share a CU (two waves per SIMD from independent workgroups: one's barrier
// and softmax stalls overlap the other's MFMAs), and the small LDS footprint
// leaves room for the GEMM workgroups of concurrent streams. A 128-vector
// work item is split over 2 workgroups, or 4 or 8 of fewer waves on small
// grids; a vector's arithmetic is the same either way, so results do not
// depend on the batch. (With 32-key tiles and one 8-wave workgroup per CU the
// text batch of 64 rows ran 2.5 % slower.)
//  * K and V tiles go from HBM/L2 straight into LDS with
//    buffer_load_dwordx4 ... lds (one instruction moves 1 KB = 256 / HD
//    rows), double buffered: tile t+1 is in flight while tile t is
//    consumed; one barrier per tile. The whole byte offset of a key row
//    (tile start included) is the instruction's range-checked vector offset,
//    so keys past the row end fall outside the buffer window and read as
//    zero, whatever memory follows the row.
//  * S^T = K . Q^T per 16-key block: K rows are stored with their 16-byte
//    chunks XOR-swizzled by (key % 16), so the 16 key rows read at one chunk
//    hit 16 distinct bank groups. Lane l holds keys 4 (l / 16) + r of each
//    block for query vector l % 16; max and sum reduce over the four lanes
//    of a query.
//  * O^T += V^T . P^T: MFMA r of a key block sums keys 4 g + r (g = lane /
//    16), exactly the probabilities lane g holds in register r; lane l reads
//    V row 4 g + r at dims 64 c + 4 (l % 16) .. + 3, one dim for each of the
//    four output tiles 4 c + t (tile row i = head dim 64 c + 4 i + t). V rows
//    are read contiguously by each 16-lane group and stay unswizzled.
//  * Online softmax in log2 units (v_exp_f32) with a lazily moved reference
//    max, so the output accumulators are rescaled only when a query's running
//    max grows by more than 2^8.
// max / sum of v over lanes l, l ^ 16, l ^ 32 and l ^ 48 through the VALU
// lane swaps v_permlane16_swap and v_permlane32_swap (no LDS round trip as
// with ds_bpermute). Each swap of v with itself leaves {v[l], v[l ^ 16]}
// (resp. {v[l], v[l ^ 32]}) in the two results, so folding them gives the
// same value, bit for bit, as v op __shfl_xor(v, 16) (resp. 32).
__device__ __forceinline__ float fold_xor16_32_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float fold_xor16_32_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Head dims above 256 (512: the global layers of the reference manifest) split
// each 16-vector group's dims over DS = HD / 256 waves: every wave holds its
// 256 dims of the queries and of the output, computes the scores' partial sums
// over them, and the DS partial sums of a score meet through LDS (added in
// dim-block order, so every wave of a group holds the same bits); the softmax
// is then repeated identically in each wave, which applies P to its own dims of
// V. Register use per wave is that of head_dim 256.
template <int HD>
constexpr int attn_dim_split() { return HD > 256 ? HD / 256 : 1; }

// Short grids (a few rows of a few hundred tokens) leave most SIMDs idle, and
// each wave's time is its dependent MFMA work: per 16-key tile, HD / 4 score
// MFMAs and HD / 4 P.V MFMAs. With OS > 1 the OS waves of a group share one
// 16-vector group: the scores' NP partial sums (below) are split over them
// (NP / OS chains each) and meet through LDS, every wave then holds the same
// score bits and runs the same softmax, and each applies P to its own HD / OS
// dims of V. A wave's chain is HD / (4 OS) + HD / (4 OS) MFMAs per tile, and
// every score and output element is the sum it is with OS = 1.

// Every score is the sum of NP partial dot products over consecutive blocks
// of HD / NP dims (dims 0 .. HD / NP - 1 first), each a chain of HD / (4 NP)
// MFMAs from zero, folded left to right: the same bits whether one wave runs
// all NP chains or the OS waves of a group run NP / OS each and meet through
// LDS. NP depends on the head dim only (head dims above 256 split their dims
// over waves instead, with the partial sums of those waves folded the same
// way).
template <int HD>
constexpr int attn_score_parts() { return HD == 256 ? 4 : HD == 128 ? 2 : 1; }

template <int HD, int WAVES, int NS>
constexpr int attn_min_blocks() { return HD <= 256 && WAVES == 4 && NS == 2 ? 2 : 1; }

// With xcd_chunks, workgroup b runs entry start(x) + local of the work list,
// x = b % 8 (the XCD the hardware dispatches it to), local = b / 8: each XCD
// takes one contiguous eighth of the list. Consecutive work items of a row
// then share one L2, which matters when a sliding window gives neighbouring
// query blocks overlapping key ranges that differ from the rest of the row.
__device__ __forceinline__ int xcd_chunk(int b, int n) {
    const int x = b & 7, local = b >> 3, q = n >> 3, r = n & 7;
    return x * q + min(x, r) + local;
}

template <int HD, int WAVES, int KT, int OS = 1, int NS = 2>
__global__ __launch_bounds__(64 * WAVES, (attn_min_blocks<HD, WAVES, NS>())) void attn16_kernel(AttnArgs p, int xcd_chunks) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int DS = attn_dim_split<HD>();  // waves per 16-vector group (score dims)
    constexpr int HDW = HD / DS;              // head dims per wave (scores)
    constexpr int HDO = HDW / OS;             // output dims per wave
    constexpr int NKB = KT / 16;              // 16-key blocks per tile
    constexpr int NP = DS > 1 ? 1 : attn_score_parts<HD>();  // partial sums per score
    constexpr int PPW = NP / OS;              // partial sums per wave
    constexpr int CPW = HDW / 16 / OS;        // 16-dim Q chunks per wave
    constexpr int CPB = CPW / PPW;            // chunks per partial sum
    constexpr int VPW = 16 * WAVES / (DS * OS);  // query vectors per workgroup
    constexpr int SPLIT = 128 / VPW;          // workgroups per 128-vector work item
    constexpr int INSTR_PER_WAVE = KT * HD / 256 / WAVES;  // 1 KB DMA instructions per operand
    static_assert(HD == 64 || HD == 128 || HD == 256 || HD == 512, "head dim");
    static_assert(WAVES == 1 || WAVES == 2 || WAVES == 4 || WAVES == 8, "waves");
    static_assert(WAVES % (DS * OS) == 0 && 128 % VPW == 0, "vector groups");
    static_assert(OS == 1 || (DS == 1 && HDO % 64 == 0), "output split");
    static_assert(NP % OS == 0 && CPW % PPW == 0 && CPB >= 1, "score partial sums");
    static_assert(KT % 16 == 0 && INSTR_PER_WAVE >= 1 && (KT * HD / 256) % WAVES == 0, "key tile");
    static_assert(NS >= 2 && NS <= 4 && (NS - 2) * 2 * INSTR_PER_WAVE < 64, "pipeline depth");
    // One LDS object per stage, addressed with compile-time stage indices:
    // the compiler can then see that the DMA filling one stage does not alias
    // the reads of another and need not drain it before reading.
    __shared__ float Ks0[KT * HD], Ks1[KT * HD], Ks2[NS > 2 ? KT * HD : 4], Ks3[NS > 3 ? KT * HD : 4];
    __shared__ float Vs0[KT * HD], Vs1[KT * HD], Vs2[NS > 2 ? KT * HD : 4], Vs3[NS > 3 ? KT * HD : 4];
    auto kstage = [&](auto st) -> float * {
        constexpr int i = decltype(st)::value;
        if constexpr (i == 0) return Ks0;
        else if constexpr (i == 1) return Ks1;
        else if constexpr (i == 2) return Ks2;
        else return Ks3;
    };
    auto vstage = [&](auto st) -> float * {
        constexpr int i = decltype(st)::value;
        if constexpr (i == 0) return Vs0;
        else if constexpr (i == 1) return Vs1;
        else if constexpr (i == 2) return Vs2;
        else return Vs3;
    };
    // partial scores: of each wave (DS > 1), of each group's NP blocks (OS > 1)
    __shared__ f32x4 Sx[DS > 1 ? WAVES * NKB * 64 : OS > 1 ? WAVES / OS * NP * NKB * 64 : 1];

    const int wg = xcd_chunks ? xcd_chunk((int)blockIdx.x, (int)gridDim.x) : (int)blockIdx.x;
    const AttnTile tile = p.tiles[wg / SPLIT];
    const int G = p.nh / p.nkv;
    // a scalar wave index: the DMA's LDS destinations (M0) then need no
    // v_readfirstlane per instruction
    const int lane = threadIdx.x & 63, wave = uniform((int)threadIdx.x >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int dpart = DS > 1 ? wave % DS : 0;  // this wave's block of head dims
    const int opart = OS > 1 ? wave % OS : 0;  // this wave's block of output dims
    const int group = wave / (DS * OS);
    const int nvec = tile.len * G;
    const int vbase = tile.qv0 + (wg % SPLIT) * VPW;
    if (vbase >= nvec) return;   // the whole workgroup: a part past the row's vectors
    const int v = vbase + group * 16 + l16;
    const bool vvalid = v < nvec;
    const int vq = vvalid ? v : nvec - 1;
    const int qpos = vq / G;
    const int qhead = tile.kvh * G + (vq - qpos * G);
    // this wave's score dims: block dpart of the head, and within it the
    // OS-th part opart (the wave's NP / OS partial sums)
    const int sdim0 = dpart * HDW + opart * 16 * CPW;
    const float *qrow = p.q + (int64_t)(tile.tok0 + qpos) * p.ldq + qhead * HD + sdim0;

    // Query fragments pre-scaled by scale * log2(e): S^T comes out in log2
    // units. Fragment c holds dims 16 c + 4 (lane / 16) .. + 3 of the wave's
    // score dims.
    const float scale2 = p.scale * 1.4426950408889634f;
    f32x4 qf[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) qf[c] = *(const f32x4 *)(qrow + 16 * c + 4 * g) * scale2;

    f32x4 o[HDO / 16];
#pragma unroll
    for (int t = 0; t < HDO / 16; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_ref = -INFINITY, l_run = 0.f;

    const int v_last = min(vbase + VPW, nvec) - 1;
    const int p_lo = vbase / G, p_hi = v_last / G;
    int k_lo = 0, k_hi = tile.len - 1;
    if (p.window >= 0) {
        k_lo = max(0, p_lo - p.window);
        k_hi = min(tile.len - 1, p_hi + p.window);
    }
    const int k_first = (k_lo / KT) * KT;
    const int n_tiles = (k_hi - k_first) / KT + 1;

    // Buffer windows over this row's keys of this KV head.
    const int ldk = (int)p.ldk, ldv = (int)p.ldv;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.k + (int64_t)tile.tok0 * p.ldk + tile.kvh * HD), (short)0,
        ((tile.len - 1) * ldk + HD) * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.v + (int64_t)tile.tok0 * p.ldv + tile.kvh * HD), (short)0,
        ((tile.len - 1) * ldv + HD) * 4, 0x00020000);
    // DMA instruction j of a tile moves floats 256 j .. 256 j + 255 of the
    // tile (1 KB: 256 / HD rows, or 1 / (HD / 256) of a row): lane l fills
    // chunk slot s of row r for float e = 256 j + 4 l = r HD + 4 s (K: with
    // global chunk s ^ (r % 16)).
    int koff[INSTR_PER_WAVE], voff[INSTR_PER_WAVE];
#pragma unroll
    for (int q = 0; q < INSTR_PER_WAVE; ++q) {
        const int e = (wave * INSTR_PER_WAVE + q) * 256 + 4 * lane;
        const int r = e / HD;
        const int slot = (e % HD) / 4;
        koff[q] = (r * ldk + 4 * (slot ^ (r & 15))) * 4;
        voff[q] = (r * ldv + 4 * slot) * 4;
    }
    auto issue = [&](auto st, int k0) {
        float *kd = kstage(st);
        float *vd = vstage(st);
#pragma unroll
        for (int q = 0; q < INSTR_PER_WAVE; ++q) {
            const int f0 = (wave * INSTR_PER_WAVE + q) * 256;
            // the tile offset goes into the range-checked vector offset (the
            // scalar offset is outside the buffer's bounds check)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rk, (__attribute__((address_space(3))) void *)&kd[f0], 16,
                koff[q] + k0 * ldk * 4, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rv, (__attribute__((address_space(3))) void *)&vd[f0], 16,
                voff[q] + k0 * ldv * 4, 0, 0, 0);
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;

    issue(S0{}, k_first);
    if constexpr (NS > 2) if (1 < n_tiles) issue(S1{}, k_first + KT);
    if constexpr (NS > 3) if (2 < n_tiles) issue(S2{}, k_first + 2 * KT);
    // key tile it lives in stage it % NS; the loop is unrolled NS times so
    // the stage index is a constant
    auto step = [&](int it, auto st) {
        constexpr int cur = decltype(st)::value;
        const int k0 = k_first + it * KT;
        // this wave's DMA of tile it has landed: only the NS - 2 later tiles
        // (2 x INSTR_PER_WAVE instructions each) may still be in flight
        if (it + NS - 2 < n_tiles) wait_vmcnt<(NS - 2) * 2 * INSTR_PER_WAVE>();
        else wait_vmcnt<0>();
        __syncthreads();   // ... and every wave's; tile it - 1 is no longer read
        if (it + NS - 1 < n_tiles)
            issue(std::integral_constant<int, (cur + NS - 1) % NS>{}, k0 + (NS - 1) * KT);

        // S^T for keys kb * 16 + 4 (lane / 16) + r (register r of block kb)
        // and query vector lane % 16. K row kb * 16 + l16 holds dim chunk
        // ch = 4 c + g (of the wave's score dims: ch + sdim0 / 4) at slot
        // ch ^ l16. Chunk c adds to partial sum c / CPB. The PPW partial sums
        // advance together: step i runs chunk p * CPB + i of every partial
        // sum p, so consecutive MFMAs feed different accumulators, while each
        // partial sum still takes its chunks, and each chunk its four k, in
        // the same order (the same bits as running the sums one after
        // another). The fragments of step i + 1 are read while step i's MFMAs
        // run, and the key blocks' chains alternate.
        const float *kb0 = kstage(st) + l16 * HD;
        const int ch0 = sdim0 / 4;
        auto kfrag = [&](int c, int kb) {
            return *(const f32x4 *)(kb0 + kb * 16 * HD + 4 * ((ch0 + 4 * c + g) ^ l16));
        };
        f32x4 sp[PPW][NKB], kf[PPW][NKB];
#pragma unroll
        for (int p = 0; p < PPW; ++p)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                sp[p][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
                kf[p][kb] = kfrag(p * CPB, kb);
            }
#pragma unroll
        for (int i = 0; i < CPB; ++i) {
            f32x4 nf[PPW][NKB];
#pragma unroll
            for (int p = 0; p < PPW; ++p)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    nf[p][kb] = kf[p][kb];
                    if (i + 1 < CPB) nf[p][kb] = kfrag(p * CPB + i + 1, kb);
                }
            // keep the reads of step i + 1 ahead of step i's MFMAs
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int p = 0; p < PPW; ++p)
#pragma unroll
                    for (int kb = 0; kb < NKB; ++kb)
                        sp[p][kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            kf[p][kb][j], qf[p * CPB + i][j], sp[p][kb], 0, 0, 0);
#pragma unroll
            for (int p = 0; p < PPW; ++p)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) kf[p][kb] = nf[p][kb];
        }
        f32x4 s[NKB];
        if constexpr (DS > 1) {
            // the partial sums of the group's waves meet in LDS; the barrier
            // at the top of the next tile keeps them until all are read
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) Sx[(wave * NKB + kb) * 64 + lane] = sp[0][kb];
            __syncthreads();
            const int w0 = group * DS;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                f32x4 t = Sx[(w0 * NKB + kb) * 64 + lane];
#pragma unroll
                for (int d = 1; d < DS; ++d) t = t + Sx[((w0 + d) * NKB + kb) * 64 + lane];
                s[kb] = t;
            }
        } else if constexpr (OS > 1) {
            // the group's NP partial sums meet in LDS (same fold as below);
            // the barrier at the top of the next tile keeps them until read
#pragma unroll
            for (int i = 0; i < PPW; ++i)
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
                    Sx[((group * NP + opart * PPW + i) * NKB + kb) * 64 + lane] = sp[i][kb];
            __syncthreads();
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                f32x4 t = Sx[(group * NP * NKB + kb) * 64 + lane];
#pragma unroll
                for (int i = 1; i < NP; ++i) t = t + Sx[((group * NP + i) * NKB + kb) * 64 + lane];
                s[kb] = t;
            }
        } else {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                f32x4 t = sp[0][kb];
#pragma unroll
                for (int i = 1; i < NP; ++i) t = t + sp[i][kb];
                s[kb] = t;
            }
        }

        // Scores in log2 units; masks only on the row-tail tile and on tiles
        // that cross a sliding-window edge of some query of the block.
        // Lanes of invalid query vectors are never stored and need no mask.
        float pr[NKB][4];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) pr[kb][r] = s[kb][r];
        const bool tail = k0 + KT > tile.len;
        const bool edge = p.window >= 0 && (k0 < p_hi - p.window || k0 + KT - 1 > p_lo + p.window);
        if (tail || edge) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + kb * 16 + 4 * g + r;
                    const int dist = qpos > key ? qpos - key : key - qpos;
                    const bool ok = (key < tile.len) & ((p.window < 0) | (dist <= p.window));
                    pr[kb][r] = ok ? pr[kb][r] : -INFINITY;
                }
        }
        float tmax = pr[0][0];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, pr[kb][r]);
        tmax = fold_xor16_32_max(tmax);
        // Lazy rescale: the reference max m_ref only moves when a query's
        // max grows by more than RESCALE_LOG2 (probabilities then stay below
        // 2^RESCALE_LOG2). O and l are divided out at the end, so the result
        // is the same softmax; the 64 accumulator registers are rescaled
        // only on the (rare, wave-uniform) tiles where some max jumped.
        const bool grow = tmax > m_ref + RESCALE_LOG2;
        if (__ballot(grow)) {
            const float m_new = grow ? tmax : m_ref;
            const float alpha = m_ref == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_ref - m_new);
            l_run *= alpha;
#pragma unroll
            for (int t = 0; t < HDO / 16; ++t) o[t] = o[t] * alpha;
            m_ref = m_new;
        }
        float psum = 0.f;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[kb][r] = pr[kb][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(pr[kb][r] - m_ref);
                psum += pr[kb][r];
            }
        psum = fold_xor16_32_sum(psum);
        l_run += psum;

        // O^T += V^T P^T, keys 4 (lane / 16) + r of block kb in MFMA r: lane
        // l supplies V row kb * 16 + 4 (l / 16) + r, dims 64 c + 4 (l % 16)
        // .. + 3 of the wave's block, one per output tile 4 c + t (tile row
        // i = dim 64 c + 4 i + t).
        const float *vb = vstage(st) + 4 * g * HD + 4 * l16 + dpart * HDW + opart * HDO;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < HDO / 64; ++c) {
                    const f32x4 va = *(const f32x4 *)(vb + (kb * 16 + r) * HD + 64 * c);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        o[4 * c + t] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[t], pr[kb][r],
                                                                          o[4 * c + t], 0, 0, 0);
                }
    };
    for (int it = 0; it < n_tiles; it += NS) {
        step(it, S0{});
        if (it + 1 < n_tiles) step(it + 1, S1{});
        if constexpr (NS > 2) if (it + 2 < n_tiles) step(it + 2, S2{});
        if constexpr (NS > 3) if (it + 3 < n_tiles) step(it + 3, S3{});
    }

    if (vvalid) {
        // lane l holds, for its query vector, dims 64 c + 16 (l / 16) + 4 r
        // + t in register r of tile 4 c + t
        const float inv = 1.0f / l_run;
        float *orow = p.out + (int64_t)(tile.tok0 + qpos) * p.ldo + qhead * HD + dpart * HDW + opart * HDO;
        bool ok = isfinite(inv);
#pragma unroll
        for (int c = 0; c < HDO / 64; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                f32x4 d;
#pragma unroll
                for (int t = 0; t < 4; ++t) d[t] = o[4 * c + t][r] * inv;
                ok = ok && finite4(d);
                *(f32x4 *)(orow + 64 * c + 16 * g + 4 * r) = d;
            }
        if (!ok) raise_flag(p.flag, FLAG_NONFINITE);
    }
#endif
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
    return (hd == 64 || hd == 128 || hd == 256 || hd == 512) ? 32 * ATTN_WAVES : 0;
}

// 16x16x4 kernel with one key-tile width per head dim (so a vector's
// arithmetic never depends on the launch): 16 keys at head_dim 256 (64 KB
// double buffered, two 4-wave workgroups per CU), 32 at 128 and at 64 (the
// vision tower: 31.4 ms per 4 images against 31.8 with 64-key and 32.5 with
// 16-key tiles). At head_dim 128 and 256, grids of up to 64 work items split
// every item over 8 workgroups whose 16-vector group takes OS waves that
// split the output dims (4 at head_dim 256, 2 at 128); larger grids run two
// 4-wave workgroups per item. Other head dims split grids of fewer than 128
// items over 4 or 8 workgroups of fewer waves. Per layer, the 1 x 128-token
// row's attention (3 items) went from 24.0 to 17.6 us, a 754-token row's
// from 124 to 83 us. Two LDS stages: with the partial sums interleaved, a timing
// harness put the 128-token row at 11.1 us against 11.5 us for three stages,
// and the one-row forward went from 1.822 to 1.811 ms (two A/B pairs).
// Workgroups go to XCDs in contiguous chunks of the work list when a sliding
// window is narrower than every row (the 8 x 2048-token batch's sliding
// layers: 0.42 against 0.54 ms per launch). Every work item then spans about
// the same number of keys, so equal chunks are equal work. Rows within the
// window read the whole row from every block, where the default interleaving
// is as fast, and a list of unequal items keeps its longest-first order
// spread over all XCDs.
template <int HD, int KT>
static hipError_t launch_attn16(const AttnArgs &a, hipStream_t s) {
    // a work item is 128 query vectors: 8 groups of 16, each group one wave
    // (DS waves above head_dim 256)
    constexpr int DS = attn_dim_split<HD>();
    const int64_t t = a.n_tiles;
    const int chunks = a.window >= 0 && a.shortest > a.window + 1;
    if constexpr (DS == 1 && HD >= 128) {
        // Up to 64 items, 8 workgroups of OS waves per item fill at most the
        // 512 two-per-CU slots once; above that, two 4-wave workgroups per item
        // (the 4 x 754-token audio prompts, 72 items: 116 against 122 us for
        // four 2-wave workgroups per item; 36 items: 71 against 77 us for
        // 8 workgroups of OS = 2 waves).
        constexpr int OS = HD / 64 >= 4 ? 4 : HD / 64;
        if (8 * t <= 512)
            hipLaunchKernelGGL((attn16_kernel<HD, OS, KT, OS, 2>), dim3((unsigned)(8 * t)),
                               dim3(64 * OS), 0, s, a, chunks);
        else
            hipLaunchKernelGGL((attn16_kernel<HD, 4, KT>), dim3((unsigned)(2 * t)), dim3(256), 0,
                               s, a, chunks);
    } else if (2 * t >= 256)
        hipLaunchKernelGGL((attn16_kernel<HD, 4 * DS, KT>), dim3((unsigned)(2 * t)),
                           dim3(256 * DS), 0, s, a, chunks);
    else if (4 * t >= 256)
        hipLaunchKernelGGL((attn16_kernel<HD, 2 * DS, KT>), dim3((unsigned)(4 * t)),
                           dim3(128 * DS), 0, s, a, chunks);
    else
        hipLaunchKernelGGL((attn16_kernel<HD, DS, KT>), dim3((unsigned)(8 * t)), dim3(64 * DS),
                           0, s, a, chunks);
    return hipGetLastError();
}

// Kernel choice forced by set_attention_path (0: by shape).
static std::atomic<int> g_attention_path{ATTN_PATH_AUTO};

void set_attention_path(int path) { g_attention_path.store(path, std::memory_order_relaxed); }

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
    if (a.tokens <= 0) return hipSuccess;
    const dim3 block(64 * ATTN_WAVES);
    const int path = g_attention_path.load(std::memory_order_relaxed);
    if (path == ATTN_PATH_GENERIC) {
        if (!a.pos || !a.rowlen || a.max_len <= 0 || a.max_len > ATTN_SIMPLE_MAX_KEYS)
            return hipErrorInvalidValue;
        hipLaunchKernelGGL(attn_simple_kernel, dim3((unsigned)(a.tokens * a.nh)), dim3(64), 0, s,
                           a);
        return hipGetLastError();
    }
    // Buffer windows are per row: the longest row bounds the offsets.
    // A tail tile addresses up to 31 keys past the row end (read as zero).
    const int64_t rows = (a.max_len > 0 ? a.max_len : a.tokens) + 32;
    const bool dma = path == ATTN_PATH_AUTO &&
                     rows * std::max(std::max(a.ldk, a.ldv), (int64_t)a.hd) * 4 < INT32_MAX;
    switch (a.hd) {
        case 64:
            if (dma) return launch_attn16<64, 32>(a, s);
            hipLaunchKernelGGL((attn_mfma_kernel<64, ATTN_WAVES>), dim3(a.n_tiles), block, 0, s, a);
            return hipGetLastError();
        case 128:
            if (dma) return launch_attn16<128, 32>(a, s);
            hipLaunchKernelGGL((attn_mfma_kernel<128, ATTN_WAVES>), dim3(a.n_tiles), block, 0, s, a);
            return hipGetLastError();
        case 256:
            if (dma) return launch_attn16<256, 16>(a, s);
            hipLaunchKernelGGL((attn_mfma_kernel<256, ATTN_WAVES>), dim3(a.n_tiles), block, 0, s, a);
            return hipGetLastError();
        case 512:
            if (dma) return launch_attn16<512, 16>(a, s);
            // a row whose buffer window would pass 2 GiB (only strides of 128
            // or more KV heads get there) takes the generic kernel
            if (!a.pos || !a.rowlen || a.max_len <= 0 || a.max_len > ATTN_SIMPLE_MAX_KEYS)
                return hipErrorInvalidValue;
            hipLaunchKernelGGL(attn_simple_kernel, dim3((unsigned)(a.tokens * a.nh)), dim3(64), 0,
                               s, a);
            return hipGetLastError();
        default:
            if (!a.pos || !a.rowlen) return hipErrorInvalidValue;
            hipLaunchKernelGGL(attn_simple_kernel, dim3((unsigned)(a.tokens * a.nh)), dim3(64), 0,
                               s, a);
            return hipGetLastError();
    }
}

}  // namespace svl
