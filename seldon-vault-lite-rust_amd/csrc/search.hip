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
// streamed once per block of QB queries. A workgroup owns 256 chunks (one
// per lane) and QB queries; each step stages a 256 x 32 slice of V in LDS
// (padded rows, conflict-free column reads) and the queries' 32 x QB slice
// as doubles (broadcast reads), then every lane runs 32 x QB FMAs.
//
// Ranking: scores become 64-bit keys ordered like f64::total_cmp reversed
// (ascending key = descending score); masked-out chunks get the largest key.
// A stable device-wide radix sort by key, then a stable sort by query index,
// yields each query's ranking with ties in ascending chunk-id order.
#include <rocprim/device/device_radix_sort.hpp>

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

template <int QB>
__global__ __launch_bounds__(256) void cosine_keys_kernel(
    const float *__restrict__ V, const double *__restrict__ cnorm, const float *__restrict__ Q,
    const double *__restrict__ qnorm, int nq, int64_t n, int D, const uint8_t *__restrict__ mask,
    int64_t mask_stride, const int64_t *__restrict__ perm, uint64_t *__restrict__ keys) {
    __shared__ float vt[SEARCH_CHUNKS][SEARCH_DK + 1];
    __shared__ double qs[SEARCH_DK][QB];
    const int t = threadIdx.x;
    const int64_t c0 = (int64_t)blockIdx.x * SEARCH_CHUNKS;
    const int q0 = blockIdx.y * QB;
    double acc[QB];
#pragma unroll
    for (int j = 0; j < QB; ++j) acc[j] = 0.0;
    for (int d0 = 0; d0 < D; d0 += SEARCH_DK) {
        const int dk = min(SEARCH_DK, D - d0);
        // V slice: 256 rows x 32 columns, 16 consecutive threads per two rows
        for (int i = t; i < SEARCH_CHUNKS * SEARCH_DK; i += 256) {
            const int r = i / SEARCH_DK, k = i % SEARCH_DK;
            float v = 0.0f;
            if (c0 + r < n && k < dk) v = V[(c0 + r) * D + d0 + k];
            vt[r][k] = v;
        }
        for (int i = t; i < SEARCH_DK * QB; i += 256) {
            const int k = i / QB, j = i % QB;
            double v = 0.0;
            if (q0 + j < nq && k < dk) v = (double)Q[(int64_t)(q0 + j) * D + d0 + k];
            qs[k][j] = v;
        }
        __syncthreads();
        for (int k = 0; k < dk; ++k) {
            const double v = (double)vt[t][k];
#pragma unroll
            for (int j = 0; j < QB; ++j) acc[j] = fma(qs[k][j], v, acc[j]);
        }
        __syncthreads();
    }
    const int64_t c = c0 + t;
    if (c >= n) return;
    const double cn = cnorm[c];
    const int64_t orig = mask ? perm[c] : 0;
#pragma unroll
    for (int j = 0; j < QB; ++j) {
        const int q = q0 + j;
        if (q >= nq) break;
        uint64_t key = ~0ull;
        if (!mask || mask[(int64_t)q * mask_stride + orig])
            key = descending_key(acc[j] / (qnorm[q] * cn));
        keys[(int64_t)q * n + c] = key;
    }
}

// One lane per query: the squared norm in d order (vector.rs:33-40).
__global__ __launch_bounds__(64) void query_norm_kernel(const float *Q, int nq, int D,
                                                        double *qnorm, int *flags) {
    const int q = blockIdx.x * 64 + threadIdx.x;
    if (q >= nq) return;
    double sum = 0.0;
    int f = 0;
    for (int d = 0; d < D; ++d) {
        const float v = Q[(int64_t)q * D + d];
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
    hipLaunchKernelGGL(query_norm_kernel, dim3((unsigned)((nq + 63) / 64)), dim3(64), 0, s, Q, nq,
                       D, qnorm, flags);
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

hipError_t launch_cosine_keys(const float *V, const double *cnorm, const float *Q,
                              const double *qnorm, int nq, int64_t n, int D, const uint8_t *mask,
                              int64_t mask_stride, const int64_t *perm, uint64_t *keys,
                              hipStream_t s) {
    if (nq <= 0 || n <= 0) return hipSuccess;
    if (D <= 0) return hipErrorInvalidValue;
    const unsigned gx = (unsigned)((n + SEARCH_CHUNKS - 1) / SEARCH_CHUNKS);
#define COS_LAUNCH(QB)                                                                        \
    hipLaunchKernelGGL(cosine_keys_kernel<QB>, dim3(gx, (unsigned)((nq + QB - 1) / QB)),   \
                       dim3(256), 0, s, V, cnorm, Q, qnorm, nq, n, D, mask, mask_stride, perm, \
                       keys)
    if (nq == 1) COS_LAUNCH(1);
    else if (nq <= 4) COS_LAUNCH(4);
    else if (nq <= 8) COS_LAUNCH(8);
    else if (nq <= 16) COS_LAUNCH(16);
    else COS_LAUNCH(32);
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
