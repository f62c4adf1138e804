// Exact cosine ranking of stored chunk embeddings (src/index/vector.rs:17-97)
// for a batch of queries.
//
// Scores are the reference's bits: each (query, chunk) pair is one lane that
// accumulates dot = sum q[d] * v[d] over d = 0, 1, ..., D - 1 in double, in
// that order. A float * float product is exact in double, so the fused
// multiply-add rounds exactly once per step like the reference's separate
// multiply and add. score = dot / (query_norm * chunk_norm) with both norms
// computed in the reference's order on the host.
//
// Layout: the chunk matrix V [n, D] (rows in ascending chunk-id order) is
// streamed once per block of QB queries, a slice of 32 dimensions of the
// workgroup's chunks at a time through LDS. Blocks of 16 to 64 queries run on
// the FP64 matrix cores (cosine_keys_mfma_kernel, whose instructions add their
// four products in order); other counts run one lane per (query, chunk) pair
// with 32 FMAs per slice, whose query operands are uniform loads from a
// d-major double copy of the queries (cosine_keys_kernel).
//
// Ranking: scores become 64-bit keys ordered like f64::total_cmp reversed
// (ascending key = descending score); masked-out chunks get the largest key.
// A stable device-wide radix sort by key, then a stable sort by query index,
// yields each query's ranking with ties in ascending chunk-id order.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_segmented_radix_sort.hpp>

#include "dev_common.hpp"
#include "svl_internal.hpp"

namespace svl {

constexpr int SEARCH_CHUNKS = 256;  // chunks per workgroup (one per lane)
constexpr int SEARCH_DK = 32;       // d-slice staged per step

__device__ __forceinline__ uint64_t descending_key(double s) {
    const uint64_t b = (uint64_t)__double_as_longlong(s);
    // f64::total_cmp order as an unsigned integer, then reversed
    const uint64_t asc = (b >> 63) ? ~b : (b | 0x8000000000000000ull);
    return ~asc;
}

// Queries as doubles, d-major: Qd[d * nq_pad + q] (zero padding), so that a
// workgroup's QB query values at one d are one uniform (scalar) load.
__global__ __launch_bounds__(256) void queries_f64_kernel(const float *Q, int nq, int D,
                                                          int nq_pad, double *Qd) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)D * nq_pad) return;
    const int d = (int)(i / nq_pad), q = (int)(i % nq_pad);
    Qd[i] = q < nq ? (double)Q[(int64_t)q * D + d] : 0.0;
}

// The workgroup's QB queries are split over its waves, QW per wave: wave w
// serves chunk group w / (QB / QW) (64 * CPL chunks, CPL per lane) and query
// sub-block w % (QB / QW). A workgroup owns CH = 64 * CPL * 4 / (QB / QW)
// chunks, so HBM traffic stays one pass over V per QB queries while each
// wave needs only QW query values per step, each reused for CPL chunks
// (the uniform query loads, not the FMAs, bound the rate when CPL = 1).
template <int QB, int QW, int CPL, bool VEC4>
__global__ __launch_bounds__(256) void cosine_keys_kernel(
    const float *__restrict__ V, const double *__restrict__ cnorm,
    const double *__restrict__ Qd, int nq_pad, const double *__restrict__ qnorm, int nq,
    int64_t n, int D, const uint8_t *__restrict__ mask, int64_t mask_stride,
    const int64_t *__restrict__ perm, uint64_t *__restrict__ keys) {
    constexpr int SPLIT = QB / QW;
    static_assert(QB % QW == 0 && 4 % SPLIT == 0, "query sub-blocks must tile the 4 waves");
    constexpr int CH = 64 * CPL * 4 / SPLIT;
    __shared__ float vt[CH][SEARCH_DK + 1];
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lane = t & 63;
    const int row0 = (wave / SPLIT) * 64 * CPL + lane;   // rows row0 + 64 * i
    const int64_t c0 = (int64_t)blockIdx.x * CH;
    const int qs = blockIdx.y * QB + (wave % SPLIT) * QW;
    double acc[CPL][QW];
#pragma unroll
    for (int i = 0; i < CPL; ++i)
#pragma unroll
        for (int j = 0; j < QW; ++j) acc[i][j] = 0.0;
    // D % 4 == 0: the slice is loaded as float4, 8 lanes per row (128
    // contiguous bytes of one chunk per 8 lanes), into registers one slice
    // ahead, so the next slice's loads are in flight while this one's FMAs run
    constexpr int NPF = CH * (SEARCH_DK / 4) / 256;
    static_assert(!VEC4 || CH * (SEARCH_DK / 4) % 256 == 0, "slice tiling");
    float4 pf[VEC4 ? NPF : 1];
    auto prefetch = [&](int d0) {
#pragma unroll
        for (int j = 0; j < NPF; ++j) {
            const int i = t + 256 * j, r = i / (SEARCH_DK / 4), k = 4 * (i % (SEARCH_DK / 4));
            pf[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (c0 + r < n && d0 + k < D)
                pf[j] = *reinterpret_cast<const float4 *>(V + (c0 + r) * D + d0 + k);
        }
    };
    if (VEC4) prefetch(0);
    for (int d0 = 0; d0 < D; d0 += SEARCH_DK) {
        const int dk = min(SEARCH_DK, D - d0);
        if (VEC4) {
#pragma unroll
            for (int j = 0; j < NPF; ++j) {
                const int i = t + 256 * j, r = i / (SEARCH_DK / 4), k = 4 * (i % (SEARCH_DK / 4));
                vt[r][k] = pf[j].x;
                vt[r][k + 1] = pf[j].y;
                vt[r][k + 2] = pf[j].z;
                vt[r][k + 3] = pf[j].w;
            }
        } else {
            for (int i = t; i < CH * SEARCH_DK; i += 256) {
                const int r = i / SEARCH_DK, k = i % SEARCH_DK;
                float v = 0.0f;
                if (c0 + r < n && k < dk) v = V[(c0 + r) * D + d0 + k];
                vt[r][k] = v;
            }
        }
        __syncthreads();
        if (VEC4 && d0 + SEARCH_DK < D) prefetch(d0 + SEARCH_DK);
        const double *qrow = Qd + (int64_t)d0 * nq_pad + qs;
        for (int k = 0; k < dk; ++k) {
            const double *qk = qrow + (int64_t)k * nq_pad;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const double v = (double)vt[row0 + 64 * i][k];
#pragma unroll
                for (int j = 0; j < QW; ++j) acc[i][j] = fma(qk[j], v, acc[i][j]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int64_t c = c0 + row0 + 64 * i;
        if (c >= n) break;
        const double cn = cnorm[c];
        const int64_t orig = mask ? perm[c] : 0;
#pragma unroll
        for (int j = 0; j < QW; ++j) {
            const int q = qs + j;
            if (q >= nq) break;
            uint64_t key = ~0ull;
            if (!mask || mask[(int64_t)q * mask_stride + orig])
                key = descending_key(acc[i][j] / (qnorm[q] * cn));
            keys[(int64_t)q * n + c] = key;
        }
    }
}

// The same keys on the FP64 matrix cores, for query blocks of QB = 16 NQB
// queries (16, 32 or 64) and dimensions that are a multiple of 4.
// v_mfma_f64_16x16x4f64 adds its four products to the accumulator one after
// another in k order, rounding each sum (checked bit for bit on a million
// random outputs against a chain of FMAs; the product of two floats is exact
// in double, so only the order of the additions can matter). Instruction s of
// a staged slice takes dims d0 + 4s .. d0 + 4s + 3 as k = 0 .. 3, so every
// score is still the sum over d = 0, 1, ..., D - 1 in that order, bit for bit.
//  * A operand = queries: lane l holds query l % 16 at dim 4s + l / 16; B
//    operand = chunks: lane l holds chunk l % 16 at the same dim. Both are
//    staged in LDS as floats (queries from a d-major float copy) and widened
//    on read, which is exact. Accumulator register r of lane l is query
//    l / 16 + 4 r against chunk l % 16, so one store instruction writes 16
//    consecutive chunks (128 bytes) of four queries' key rows.
//  * Each wave owns 16 NCB chunks of the workgroup's 64 NCB and every query
//    of the block. The next slice's chunk and query values are loaded into
//    registers while the current slice's MFMAs run. Registers are bounded
//    for four waves per SIMD (the accumulators take 8 NQB NCB of them).
//  * Dims past D inside the last slice are never read (the loop stops at the
//    last group of 4); chunks past n and queries past nq read zeros and are
//    not stored.
constexpr int SEARCH_MFMA_DK = 32;

template <int NQB, int NCB>
__global__ __launch_bounds__(256, 4) void cosine_keys_mfma_kernel(
    const float *__restrict__ V, const double *__restrict__ cnorm,
    const float *__restrict__ Qf, int nq_pad, const double *__restrict__ qnorm, int nq,
    int64_t n, int D, const uint8_t *__restrict__ mask, int64_t mask_stride,
    const int64_t *__restrict__ perm, uint64_t *__restrict__ keys) {
    constexpr int QB = 16 * NQB, CH = 64 * NCB, DK = SEARCH_MFMA_DK;
    // row pitches (floats): 16 rows x 4 dims of a fragment read hit 64 banks
    constexpr int VP = DK + 4;
    constexpr int QP = QB + 16 > 48 ? QB + 16 : 48;
    constexpr int VF4 = CH * DK / 4 / 256;              // float4 of the chunk slice per thread
    constexpr int QN4 = DK * QB / 4;                    // float4 of the query slice
    constexpr int QF4 = (QN4 + 255) / 256;              // ... per thread
    static_assert(VF4 >= 1 && CH * DK / 4 % 256 == 0, "slice shape");
    typedef double f64x4 __attribute__((ext_vector_type(4)));
    __shared__ float vt[CH * VP];
    __shared__ float qt[DK * QP];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int64_t c0 = (int64_t)blockIdx.x * CH;
    const int qs = blockIdx.y * QB;

    f64x4 acc[NQB][NCB];
#pragma unroll
    for (int i = 0; i < NQB; ++i)
#pragma unroll
        for (int j = 0; j < NCB; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};

    float4 vr[VF4], qr[QF4];
    auto load = [&](int d0) {
#pragma unroll
        for (int i = 0; i < VF4; ++i) {
            const int idx = t + 256 * i, r = idx / (DK / 4), k = 4 * (idx % (DK / 4));
            vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (c0 + r < n && d0 + k < D)
                vr[i] = *reinterpret_cast<const float4 *>(V + (c0 + r) * D + d0 + k);
        }
#pragma unroll
        for (int i = 0; i < QF4; ++i) {
            const int idx = t + 256 * i, dd = idx / (QB / 4), q4 = 4 * (idx % (QB / 4));
            qr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (idx < QN4 && d0 + dd < D)
                qr[i] = *reinterpret_cast<const float4 *>(Qf + (int64_t)(d0 + dd) * nq_pad + qs + q4);
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int i = 0; i < VF4; ++i) {
            const int idx = t + 256 * i, r = idx / (DK / 4), k = 4 * (idx % (DK / 4));
            *reinterpret_cast<float4 *>(&vt[r * VP + k]) = vr[i];
        }
#pragma unroll
        for (int i = 0; i < QF4; ++i) {
            const int idx = t + 256 * i, dd = idx / (QB / 4), q4 = 4 * (idx % (QB / 4));
            if (idx < QN4) *reinterpret_cast<float4 *>(&qt[dd * QP + q4]) = qr[i];
        }
    };

    const float *vw = vt + (wave * 16 * NCB + l16) * VP + g;
    const float *qw = qt + g * QP + l16;
    load(0);
    for (int d0 = 0; d0 < D; d0 += DK) {
        store();
        __syncthreads();
        if (d0 + DK < D) load(d0 + DK);
        const int ng = min(DK, D - d0) / 4;
        for (int s = 0; s < ng; ++s) {
            double a[NQB], b[NCB];
#pragma unroll
            for (int i = 0; i < NQB; ++i) a[i] = (double)qw[4 * s * QP + 16 * i];
#pragma unroll
            for (int j = 0; j < NCB; ++j) b[j] = (double)vw[16 * j * VP + 4 * s];
#pragma unroll
            for (int i = 0; i < NQB; ++i)
#pragma unroll
                for (int j = 0; j < NCB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < NCB; ++j) {
        const int64_t c = c0 + wave * 16 * NCB + 16 * j + l16;
        if (c >= n) continue;
        const double cn = cnorm[c];
        const int64_t orig = mask ? perm[c] : 0;
#pragma unroll
        for (int i = 0; i < NQB; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = qs + 16 * i + g + 4 * r;
                if (q >= nq) continue;
                uint64_t key = ~0ull;
                if (!mask || mask[(int64_t)q * mask_stride + orig])
                    key = descending_key(acc[i][j][r] / (qnorm[q] * cn));
                keys[(int64_t)q * n + c] = key;
            }
    }
}

// Queries as floats, d-major (Qf[d * nq_pad + q], zero padding): the query
// operand of the matrix-core kernel, staged per slice with float4 loads.
__global__ __launch_bounds__(256) void queries_dmajor_kernel(const float *Q, int nq, int D,
                                                             int nq_pad, float *Qf) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)D * nq_pad) return;
    const int d = (int)(i / nq_pad), q = (int)(i % nq_pad);
    Qf[i] = q < nq ? Q[(int64_t)q * D + d] : 0.f;
}

// One workgroup per query: the row is staged in LDS with coalesced loads,
// then one lane accumulates the squared norm in d order (vector.rs:33-40).
__global__ __launch_bounds__(256) void query_norm_kernel(const float *Q, int nq, int D,
                                                         double *qnorm, int *flags) {
    __shared__ float row[8192];
    const int q = blockIdx.x;
    if (q >= nq) return;
    for (int d = threadIdx.x; d < D; d += 256) row[d] = Q[(int64_t)q * D + d];
    __syncthreads();
    if (threadIdx.x != 0) return;
    double sum = 0.0;
    int f = 0;
    for (int d = 0; d < D; ++d) {
        const float v = row[d];
        if (!isfinite(v)) f |= 1;
        sum = fma((double)v, (double)v, sum);
    }
    if (!isfinite(sum) || sum <= 0.0) f |= 2;
    qnorm[q] = sqrt(sum);
    flags[q] = f;
}

hipError_t launch_query_norms(const float *Q, int nq, int D, double *qnorm, int *flags,
                              hipStream_t s) {
    if (nq <= 0) return hipSuccess;
    if (D > 8192) return hipErrorInvalidValue;
    hipLaunchKernelGGL(query_norm_kernel, dim3((unsigned)nq), dim3(256), 0, s, Q, nq, D, qnorm,
                       flags);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void iota_kernel(uint32_t *v, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < count) v[i] = (uint32_t)i;
}

// query index of every sorted pair: the key of the second, stable sort
__global__ __launch_bounds__(256) void query_of_kernel(const uint32_t *idx, int64_t count,
                                                       int64_t n, uint32_t *qkey) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < count) qkey[i] = (uint32_t)(idx[i] / (uint64_t)n);
}

// Hits [offset, offset + take[q]) of each query's ranking: original chunk
// index and score, the score recovered from the pair's (unsorted) key bits.
__global__ __launch_bounds__(256) void gather_hits_kernel(const uint64_t *keys,
                                                          const uint32_t *sidx, int nq, int64_t n,
                                                          const int64_t *perm, int64_t offset,
                                                          int64_t limit, const int64_t *take,
                                                          int64_t *out_index, double *out_score) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int q = blockIdx.y;
    if (q >= nq || i >= take[q]) return;
    const uint32_t flat = sidx[(int64_t)q * n + offset + i];
    const uint64_t asc = ~keys[flat];
    const uint64_t b = (asc >> 63) ? (asc & 0x7FFFFFFFFFFFFFFFull) : ~asc;
    out_index[(int64_t)q * limit + i] = perm[flat % (uint64_t)n];
    out_score[(int64_t)q * limit + i] = __longlong_as_double((long long)b);
}

int cosine_query_block(int nq) {
    return nq == 1 ? 1 : nq <= 4 ? 4 : nq <= 8 ? 8 : nq <= 16 ? 16 : nq <= 32 ? 32 : 64;
}

hipError_t launch_cosine_keys(const float *V, const double *cnorm, const float *Q,
                              const double *qnorm, int nq, int64_t n, int D, const uint8_t *mask,
                              int64_t mask_stride, const int64_t *perm, double *Qd,
                              uint64_t *keys, hipStream_t s) {
    if (nq <= 0 || n <= 0) return hipSuccess;
    if (D <= 0) return hipErrorInvalidValue;
    const int qb = cosine_query_block(nq);
    const int nq_pad = (nq + qb - 1) / qb * qb;
    const int64_t total = (int64_t)D * nq_pad;
    const bool vec4 = D % 4 == 0;
    if (vec4 && qb >= 16) {
        // FP64 matrix cores: 128 chunks per workgroup, the whole query block;
        // the queries as floats, d-major, in the first half of Qd's space
        float *Qf = reinterpret_cast<float *>(Qd);
        hipLaunchKernelGGL(queries_dmajor_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                           0, s, Q, nq, D, nq_pad, Qf);
        const dim3 grid((unsigned)((n + 127) / 128), (unsigned)(nq_pad / qb));
        if (qb == 16)
            hipLaunchKernelGGL((cosine_keys_mfma_kernel<1, 2>), grid, dim3(256), 0, s, V, cnorm,
                               Qf, nq_pad, qnorm, nq, n, D, mask, mask_stride, perm, keys);
        else if (qb == 32)
            hipLaunchKernelGGL((cosine_keys_mfma_kernel<2, 2>), grid, dim3(256), 0, s, V, cnorm,
                               Qf, nq_pad, qnorm, nq, n, D, mask, mask_stride, perm, keys);
        else
            hipLaunchKernelGGL((cosine_keys_mfma_kernel<4, 2>), grid, dim3(256), 0, s, V, cnorm,
                               Qf, nq_pad, qnorm, nq, n, D, mask, mask_stride, perm, keys);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(queries_f64_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       Q, nq, D, nq_pad, Qd);
#define COS_LAUNCH(QB, QW, CPL)                                                               \
    do {                                                                                      \
        constexpr int CH = 64 * CPL * 4 / (QB / QW);                                          \
        const dim3 grid((unsigned)((n + CH - 1) / CH), (unsigned)(nq_pad / QB));              \
        if (vec4)                                                                             \
            hipLaunchKernelGGL((cosine_keys_kernel<QB, QW, CPL, true>), grid, dim3(256), 0, \
                               s, V, cnorm, Qd, nq_pad, qnorm, nq, n, D, mask, mask_stride,   \
                               perm, keys);                                                   \
        else                                                                                  \
            hipLaunchKernelGGL((cosine_keys_kernel<QB, QW, CPL, false>), grid, dim3(256), 0, \
                               s, V, cnorm, Qd, nq_pad, qnorm, nq, n, D, mask, mask_stride,   \
                               perm, keys);                                                   \
    } while (0)
    // (QB, QW, CPL) measured best at 1M x 768 per query count: up to 16
    // queries the pass over V (one per QB queries) bounds the rate; from 32
    // on, CPL = 2 halves the uniform query loads per FMA.
    switch (qb) {
        case 1: COS_LAUNCH(1, 1, 1); break;
        case 4: COS_LAUNCH(4, 4, 1); break;
        case 8: COS_LAUNCH(8, 2, 2); break;
        case 16: COS_LAUNCH(16, 4, 2); break;
        case 32: COS_LAUNCH(32, 8, 2); break;
        default: COS_LAUNCH(64, 16, 2); break;
    }
#undef COS_LAUNCH
    return hipGetLastError();
}

hipError_t rank_sort(const uint64_t *keys, uint64_t *keys_alt, uint32_t *idx, uint32_t *idx_alt,
                     uint32_t *qkey, int nq, int64_t n, void *tmp, size_t *tmp_bytes,
                     const uint32_t **sorted, hipStream_t s) {
    const int64_t count = (int64_t)nq * n;
    if (count > (int64_t)UINT32_MAX) return hipErrorInvalidValue;
    unsigned qbits = 1;
    while ((1ull << qbits) < (unsigned long long)nq) ++qbits;
    uint32_t *qkey_alt = reinterpret_cast<uint32_t *>(keys_alt);  // sorted keys are not kept
    if (!tmp) {
        size_t a = 0, b = 0;
        hipError_t e = rocprim::radix_sort_pairs(nullptr, a, keys, keys_alt, idx, idx_alt,
                                                 (size_t)count, 0, 64, s);
        if (e != hipSuccess) return e;
        e = rocprim::radix_sort_pairs(nullptr, b, qkey, qkey_alt, idx_alt, idx, (size_t)count, 0,
                                      qbits, s);
        *tmp_bytes = std::max(a, b);
        return e;
    }
    *sorted = idx_alt;
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(iota_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, idx,
                       count);
    hipError_t e = rocprim::radix_sort_pairs(tmp, *tmp_bytes, keys, keys_alt, idx, idx_alt,
                                             (size_t)count, 0, 64, s);
    if (e != hipSuccess || nq == 1) return e;
    // stable regroup by query index: within a query the key order survives
    hipLaunchKernelGGL(query_of_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s,
                       idx_alt, count, n, qkey);
    e = rocprim::radix_sort_pairs(tmp, *tmp_bytes, qkey, qkey_alt, idx_alt, idx, (size_t)count,
                                  0, qbits, s);
    *sorted = idx;
    return e;
}

// ---- top-K selection (offset + limit much smaller than the index) ---------------
// Ascending bitonic sort of 1024 * E keys by a block of 1024 threads, thread t
// holding elements t * E .. t * E + E - 1 in registers. With indices the
// order is (key, index) lexicographic, a total order when the indices are
// distinct. Strides below E exchange in registers, strides below 64 E across
// the wave with lane shuffles, and only the wider ones go through LDS (two
// barriers each), so a 4096-key sort takes 10 LDS stages instead of 78.
constexpr int SORT_THREADS = 1024;

template <bool WITH_IDX>
__device__ __forceinline__ bool key_less(uint64_t a, uint32_t ai, uint64_t b, uint32_t bi) {
    return a < b || (WITH_IDX && a == b && ai < bi);
}

template <int E, bool WITH_IDX, int J>
__device__ __forceinline__ void bitonic_in_thread(uint64_t (&k)[E], uint32_t (&x)[E], int size) {
    const int t = threadIdx.x;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (e & J) continue;
        const int f = e ^ J;
        const bool asc = ((t * E + e) & size) == 0;
        if (key_less<WITH_IDX>(k[f], x[f], k[e], x[e]) == asc) {
            const uint64_t tk = k[e];
            k[e] = k[f];
            k[f] = tk;
            if constexpr (WITH_IDX) {
                const uint32_t tx = x[e];
                x[e] = x[f];
                x[f] = tx;
            }
        }
    }
}

template <int E, bool WITH_IDX>
__device__ __forceinline__ void bitonic_block(uint64_t (&k)[E], uint32_t (&x)[E], uint64_t *lk,
                                              uint32_t *lx) {
    const int t = threadIdx.x;
    for (int size = 2; size <= SORT_THREADS * E; size <<= 1) {
        for (int j = size >> 1; j > 0; j >>= 1) {
            if (j < E) {
                if (j == 1) bitonic_in_thread<E, WITH_IDX, 1>(k, x, size);
                if constexpr (E > 2) if (j == 2) bitonic_in_thread<E, WITH_IDX, 2>(k, x, size);
                if constexpr (E > 4) if (j == 4) bitonic_in_thread<E, WITH_IDX, 4>(k, x, size);
                continue;
            }
            const int m = j / E;   // partner thread t ^ m
            uint64_t ok[E];
            uint32_t ox[E];
            if (j < 64 * E) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    ok[e] = __shfl_xor(k[e], m, 64);
                    if constexpr (WITH_IDX) ox[e] = __shfl_xor(x[e], m, 64);
                }
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    lk[t * E + e] = k[e];
                    if constexpr (WITH_IDX) lx[t * E + e] = x[e];
                }
                __syncthreads();
                const int p = t ^ m;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    ok[e] = lk[p * E + e];
                    if constexpr (WITH_IDX) ox[e] = lx[p * E + e];
                }
                __syncthreads();
            }
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int i = t * E + e;
                const bool want_min = ((i & j) == 0) == ((i & size) == 0);
                const uint32_t oxe = WITH_IDX ? ox[e] : 0u;
                const bool other_less = key_less<WITH_IDX>(ok[e], oxe, k[e], x[e]);
                if (other_less == want_min) {
                    k[e] = ok[e];
                    if constexpr (WITH_IDX) x[e] = oxe;
                }
            }
        }
    }
}

// One block per query: its SAMPLE_COUNT samples, every stride-th key
// (stride = n / SAMPLE_COUNT, so every sample position is below n), sorted
// ascending into sorted[q * SAMPLE_COUNT ...].
__global__ __launch_bounds__(SORT_THREADS) void sort_samples_kernel(const uint64_t *keys,
                                                                    int64_t n, int64_t stride,
                                                                    uint64_t *sorted) {
    constexpr int E = SAMPLE_COUNT / SORT_THREADS;
    __shared__ uint64_t lk[SAMPLE_COUNT];
    const int q = blockIdx.x, t = threadIdx.x;
    uint64_t k[E];
    uint32_t x[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        k[e] = keys[(int64_t)q * n + (int64_t)(t * E + e) * stride];
        x[e] = 0;
    }
    bitonic_block<E, false>(k, x, lk, nullptr);
#pragma unroll
    for (int e = 0; e < E; ++e) sorted[(int64_t)q * SAMPLE_COUNT + t * E + e] = k[e];
}

// Candidates of query q: every admitted key <= sorted sample `rank`, in
// position order. Pass 1 counts them per block of COMPACT_ITEMS keys; a
// per-query scan gives each block its offset (and cnt[q] the total); pass 2
// writes them at cand[q * cap + offset], keeping the first cap.
constexpr int COMPACT_ITEMS = 4096;  // keys per block: 256 lanes x 16

__device__ __forceinline__ bool is_candidate(uint64_t k, uint64_t thresh) {
    return k != ~0ull && k <= thresh;
}

__global__ __launch_bounds__(256) void count_candidates_kernel(const uint64_t *keys, int64_t n,
                                                               const uint64_t *sorted_samples,
                                                               int S, int rank, int nblk,
                                                               unsigned int *blk_count) {
    __shared__ unsigned int wave_total[4];
    const int q = blockIdx.y;
    const uint64_t thresh = sorted_samples[(int64_t)q * S + rank];
    const int64_t base = (int64_t)blockIdx.x * COMPACT_ITEMS;
    unsigned int c = 0;
    for (int i = threadIdx.x; i < COMPACT_ITEMS; i += 256) {
        const int64_t pos = base + i;
        if (pos < n && is_candidate(keys[(int64_t)q * n + pos], thresh)) ++c;
    }
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
    if ((threadIdx.x & 63) == 0) wave_total[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0)
        blk_count[(int64_t)q * nblk + blockIdx.x] =
            wave_total[0] + wave_total[1] + wave_total[2] + wave_total[3];
}

// One block per query: exclusive scan of its block counts (in place) and the
// total, 256 counts at a time.
__global__ __launch_bounds__(256) void scan_candidates_kernel(unsigned int *blk_count, int nblk,
                                                              unsigned int *cnt) {
    __shared__ unsigned int wave_total[4];
    const int q = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned int *c = blk_count + (int64_t)q * nblk;
    unsigned int run = 0;
    for (int b0 = 0; b0 < nblk; b0 += 256) {
        const int b = b0 + threadIdx.x;
        const unsigned int v = b < nblk ? c[b] : 0u;
        unsigned int incl = v;
        for (int o = 1; o < 64; o <<= 1) {
            const unsigned int up = __shfl_up(incl, o, 64);
            if (lane >= o) incl += up;
        }
        if (lane == 63) wave_total[wave] = incl;
        __syncthreads();
        unsigned int before = run;
        for (int w = 0; w < wave; ++w) before += wave_total[w];
        if (b < nblk) c[b] = before + incl - v;
        run += wave_total[0] + wave_total[1] + wave_total[2] + wave_total[3];
        __syncthreads();
    }
    if (threadIdx.x == 0) cnt[q] = run;
}

__global__ __launch_bounds__(256) void write_candidates_kernel(
    const uint64_t *keys, int64_t n, const uint64_t *sorted_samples, int S, int rank, int nblk,
    const unsigned int *blk_offset, int64_t cap, uint64_t *cand_key, uint32_t *cand_idx) {
    __shared__ unsigned int wave_count[4];
    const int q = blockIdx.y;
    const uint64_t thresh = sorted_samples[(int64_t)q * S + rank];
    const int64_t base = (int64_t)blockIdx.x * COMPACT_ITEMS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned int offset = blk_offset[(int64_t)q * nblk + blockIdx.x];
    // rounds of 256 consecutive keys, in position order within the block
    for (int r = 0; r < COMPACT_ITEMS; r += 256) {
        const int64_t pos = base + r + threadIdx.x;
        uint64_t k = 0;
        const bool hit = pos < n && is_candidate(k = keys[(int64_t)q * n + pos], thresh);
        const uint64_t ballot = __ballot(hit);
        if (lane == 0) wave_count[wave] = (unsigned int)__popcll(ballot);
        __syncthreads();
        unsigned int before = 0;
        for (int w = 0; w < wave; ++w) before += wave_count[w];
        const unsigned int below = (unsigned int)__popcll(ballot & ((1ull << lane) - 1));
        if (hit) {
            const int64_t slot = (int64_t)offset + before + below;
            if (slot < cap) {
                cand_key[(int64_t)q * cap + slot] = k;
                cand_idx[(int64_t)q * cap + slot] = (uint32_t)((int64_t)q * n + pos);
            }
        }
        offset += wave_count[0] + wave_count[1] + wave_count[2] + wave_count[3];
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void segment_bounds_kernel(const unsigned int *cnt, int nq,
                                                             int64_t cap, unsigned int *begin,
                                                             unsigned int *end) {
    const int q = blockIdx.x * 256 + threadIdx.x;
    if (q >= nq) return;
    begin[q] = (unsigned int)(q * cap);
    end[q] = (unsigned int)(q * cap + min((int64_t)cnt[q], cap));
}

// For a few queries, the one sample the candidate passes read (rank `rank`
// of the ascending order, written to sorted[q * SAMPLE_COUNT + rank]) by
// counting instead of sorting: block (c, q) takes samples 64 c .. 64 c + 63
// of query q, one per lane; wave w of its eight counts the samples j of its
// eighth [512 w, 512 w + 512) below the lane's sample (ties by position),
// and the sample whose eight counts sum to `rank` is the one sorted order
// puts there. 64 blocks per query spread over the CUs, where the sort is one
// block's chain of compare-exchange stages. Every thread loads its eight
// samples before storing any, and the count reads two samples per LDS read,
// eight reads in flight.
constexpr int SELECT_WAVES = 8;
__global__ __launch_bounds__(64 * SELECT_WAVES) void select_sample_kernel(const uint64_t *keys,
                                                                          int64_t n, int64_t stride,
                                                                          int rank,
                                                                          uint64_t *sorted) {
    constexpr int THREADS = 64 * SELECT_WAVES, PER_THREAD = SAMPLE_COUNT / THREADS;
    constexpr int SPAN = SAMPLE_COUNT / SELECT_WAVES;
    __shared__ __align__(16) uint64_t ls[SAMPLE_COUNT];
    __shared__ int part[SELECT_WAVES][64];
    const int q = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const uint64_t *kq = keys + (int64_t)q * n;
    uint64_t r[PER_THREAD];
#pragma unroll
    for (int e = 0; e < PER_THREAD; ++e) r[e] = kq[(int64_t)(t + e * THREADS) * stride];
#pragma unroll
    for (int e = 0; e < PER_THREAD; ++e) ls[t + e * THREADS] = r[e];
    __syncthreads();
    const int me = (int)blockIdx.x * 64 + lane;
    const uint64_t v = ls[me];
    const int j0 = w * SPAN;
    const ulonglong2 *l2 = reinterpret_cast<const ulonglong2 *>(ls + j0);
    int below = 0;
#pragma unroll 8
    for (int i = 0; i < SPAN / 2; ++i) {
        const ulonglong2 u = l2[i];
        const int j = j0 + 2 * i;
        below += (int)((u.x < v) | ((u.x == v) & (j < me)));
        below += (int)((u.y < v) | ((u.y == v) & (j + 1 < me)));
    }
    part[w][lane] = below;
    __syncthreads();
    if (w == 0) {
        int total = 0;
#pragma unroll
        for (int k = 0; k < SELECT_WAVES; ++k) total += part[k][lane];
        if (total == rank) sorted[(int64_t)q * SAMPLE_COUNT + rank] = v;
    }
}

hipError_t sort_samples(const uint64_t *keys, int nq, int64_t n, uint64_t *sorted,
                        hipStream_t s) {
    if (nq <= 0) return hipSuccess;
    hipLaunchKernelGGL(sort_samples_kernel, dim3((unsigned)nq), dim3(1024), 0, s, keys, n,
                       n / SAMPLE_COUNT, sorted);
    return hipGetLastError();
}

hipError_t select_sample(const uint64_t *keys, int nq, int64_t n, int rank, uint64_t *sorted,
                         hipStream_t s) {
    if (nq <= 0) return hipSuccess;
    if (rank < 0 || rank >= SAMPLE_COUNT) return hipErrorInvalidValue;
    hipLaunchKernelGGL(select_sample_kernel, dim3(SAMPLE_COUNT / 64, (unsigned)nq),
                       dim3(64 * SELECT_WAVES), 0, s, keys, n, n / SAMPLE_COUNT, rank, sorted);
    return hipGetLastError();
}

int candidate_blocks(int64_t n) { return (int)((n + COMPACT_ITEMS - 1) / COMPACT_ITEMS); }

hipError_t launch_compact_keys(const uint64_t *keys, int nq, int64_t n,
                               const uint64_t *sorted_samples, int S, int rank, int64_t cap,
                               unsigned int *blk_count, unsigned int *cnt, uint64_t *cand_key,
                               uint32_t *cand_idx, hipStream_t s) {
    const int nblk = candidate_blocks(n);
    const dim3 grid((unsigned)nblk, (unsigned)nq);
    hipLaunchKernelGGL(count_candidates_kernel, grid, dim3(256), 0, s, keys, n, sorted_samples, S,
                       rank, nblk, blk_count);
    hipLaunchKernelGGL(scan_candidates_kernel, dim3((unsigned)nq), dim3(256), 0, s, blk_count,
                       nblk, cnt);
    hipLaunchKernelGGL(write_candidates_kernel, grid, dim3(256), 0, s, keys, n, sorted_samples, S,
                       rank, nblk, blk_count, cap, cand_key, cand_idx);
    return hipGetLastError();
}

// Candidates of each query in (key, position) order: they are written in
// position order, so one stable segmented sort by key suffices. Results in
// key_alt / idx_alt.
hipError_t sort_candidates(const uint64_t *cand_key, const uint32_t *cand_idx, uint64_t *key_alt,
                           uint32_t *idx_alt, const unsigned int *cnt, unsigned int *begin,
                           unsigned int *end, int nq, int64_t cap, void *tmp, size_t *tmp_bytes,
                           hipStream_t s) {
    const unsigned int total = (unsigned int)(nq * cap);
    if (tmp)
        hipLaunchKernelGGL(segment_bounds_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256),
                           0, s, cnt, nq, cap, begin, end);
    return rocprim::segmented_radix_sort_pairs(tmp, *tmp_bytes, cand_key, key_alt, cand_idx,
                                               idx_alt, total, (unsigned int)nq, begin, end, 0, 64,
                                               s);
}

// Candidate lists of at most CAND_LDS entries: one block per query sorts
// (key, position) pairs, padded with all-ones to 1024 * E entries (E from the
// longest list of the launch); positions are distinct, so this is the order
// the stable key sort gives to candidates stored in position order.
template <int E>
__global__ __launch_bounds__(SORT_THREADS) void sort_candidates_lds_kernel(
    const uint64_t *cand_key, const uint32_t *cand_idx, const unsigned int *cnt, int64_t cap,
    uint64_t *key_alt, uint32_t *idx_alt) {
    __shared__ uint64_t lk[SORT_THREADS * E];
    __shared__ uint32_t lx[SORT_THREADS * E];
    const int q = blockIdx.x, t = threadIdx.x;
    const int c = (int)min<int64_t>(min<int64_t>((int64_t)cnt[q], cap), SORT_THREADS * E);
    const int64_t base = (int64_t)q * cap;
    uint64_t k[E];
    uint32_t x[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = t * E + e;
        k[e] = i < c ? cand_key[base + i] : ~0ull;
        x[e] = i < c ? cand_idx[base + i] : ~0u;
    }
    bitonic_block<E, true>(k, x, lk, lx);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int i = t * E + e;
        if (i < c) {
            key_alt[base + i] = k[e];
            idx_alt[base + i] = x[e];
        }
    }
}

hipError_t sort_candidates_lds(const uint64_t *cand_key, const uint32_t *cand_idx,
                               uint64_t *key_alt, uint32_t *idx_alt, const unsigned int *cnt,
                               int nq, int64_t cap, int64_t most, hipStream_t s) {
    if (nq <= 0) return hipSuccess;
    if (most > CAND_LDS) return hipErrorInvalidValue;
    const dim3 grid((unsigned)nq), block(SORT_THREADS);
    if (most <= SORT_THREADS)
        hipLaunchKernelGGL((sort_candidates_lds_kernel<1>), grid, block, 0, s, cand_key, cand_idx,
                           cnt, cap, key_alt, idx_alt);
    else if (most <= 2 * SORT_THREADS)
        hipLaunchKernelGGL((sort_candidates_lds_kernel<2>), grid, block, 0, s, cand_key, cand_idx,
                           cnt, cap, key_alt, idx_alt);
    else if (most <= 4 * SORT_THREADS)
        hipLaunchKernelGGL((sort_candidates_lds_kernel<4>), grid, block, 0, s, cand_key, cand_idx,
                           cnt, cap, key_alt, idx_alt);
    else
        hipLaunchKernelGGL((sort_candidates_lds_kernel<8>), grid, block, 0, s, cand_key, cand_idx,
                           cnt, cap, key_alt, idx_alt);
    return hipGetLastError();
}

// Hits from the sorted candidates: entries [offset, offset + take[q]) of
// segment q.
__global__ __launch_bounds__(256) void gather_candidates_kernel(const uint64_t *cand_key,
                                                                const uint32_t *cand_idx, int nq,
                                                                int64_t n, int64_t cap,
                                                                const int64_t *perm,
                                                                int64_t offset, int64_t limit,
                                                                const int64_t *take,
                                                                int64_t *out_index,
                                                                double *out_score) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int q = blockIdx.y;
    if (q >= nq || i >= take[q]) return;
    const int64_t src = (int64_t)q * cap + offset + i;
    const uint64_t asc = ~cand_key[src];
    const uint64_t b = (asc >> 63) ? (asc & 0x7FFFFFFFFFFFFFFFull) : ~asc;
    out_index[(int64_t)q * limit + i] = perm[cand_idx[src] % (uint64_t)n];
    out_score[(int64_t)q * limit + i] = __longlong_as_double((long long)b);
}

hipError_t launch_gather_candidates(const uint64_t *cand_key, const uint32_t *cand_idx, int nq,
                                    int64_t n, int64_t cap, const int64_t *perm, int64_t offset,
                                    int64_t limit, const int64_t *take, int64_t *out_index,
                                    double *out_score, hipStream_t s) {
    if (nq <= 0 || limit <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_candidates_kernel,
                       dim3((unsigned)((limit + 255) / 256), (unsigned)nq), dim3(256), 0, s,
                       cand_key, cand_idx, nq, n, cap, perm, offset, limit, take, out_index,
                       out_score);
    return hipGetLastError();
}

hipError_t launch_gather_hits(const uint64_t *keys, const uint32_t *sidx, int nq, int64_t n,
                              const int64_t *perm, int64_t offset, int64_t limit,
                              const int64_t *take, int64_t *out_index, double *out_score,
                              hipStream_t s) {
    if (nq <= 0 || limit <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_hits_kernel, dim3((unsigned)((limit + 255) / 256), (unsigned)nq),
                       dim3(256), 0, s, keys, sidx, nq, n, perm, offset, limit, take, out_index,
                       out_score);
    return hipGetLastError();
}

}  // namespace svl
