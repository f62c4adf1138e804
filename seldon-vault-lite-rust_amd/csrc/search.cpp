// Host runtime of the exact vector search (the svl_vector_* part of
// include/svl_hip.h): vector::rank of src/index/vector.rs:17-97 plus the
// pagination slice of Index::search (src/index/mod.rs:347-359), for a batch
// of queries against chunk embeddings resident in HBM.
//
// The index keeps the chunk matrix in ascending chunk-id order (a stable sort
// of the caller's order), so the stable ranking sort breaks score ties by
// chunk id, then by the caller's order, as the reference's stable sort_by
// does. Each chunk's norm is sqrt of its squared sum accumulated in double in
// d order, computed once here instead of per query (it does not depend on
// the query); chunks whose sum is zero or non-finite are remembered and
// reported when a query's filter admits them (vector.rs:77-82).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <memory>
#include <mutex>
#include <numeric>
#include <thread>
#include <vector>

#include "../../include/svl_hip.h"
#include "host_common.hpp"
#include "svl_internal.hpp"

namespace {

using namespace svl;

constexpr int64_t MAX_EMBEDDING_DIMENSION = 8192;  // storage/model.rs:35

}  // namespace

struct svl_vector_index {
    int device = -1;
    hipStream_t stream = nullptr;
    int64_t n = 0, D = 0;
    std::vector<uint64_t> ids;     // caller order
    std::vector<uint8_t> bad;      // caller order: zero / non-finite norm
    std::vector<int64_t> bad_list;  // caller indices with bad norms
    DevBuf<float> V;                // [n, D] chunk-id order
    DevBuf<double> cnorm;           // [n] chunk-id order
    DevBuf<int64_t> perm;           // chunk-id order -> caller index
    // per-call workspace
    DevBuf<float> Q;
    DevBuf<double> qnorm, Qd;
    DevBuf<int> qflags;
    DevBuf<uint8_t> mask;
    DevBuf<uint64_t> keys, keys_alt;
    DevBuf<uint32_t> idx, idx_alt, qkey;
    DevBuf<unsigned char> tmp;
    DevBuf<uint64_t> samples, cand_key, cand_key_alt;
    DevBuf<uint32_t> cand_idx, cand_idx_alt;
    DevBuf<unsigned int> cnt, seg_begin, seg_end, blk_count;
    DevBuf<int64_t> take, out_index;
    DevBuf<double> out_score;
    std::mutex mu;

    ~svl_vector_index() {
        if (device >= 0) (void)hipSetDevice(device);
        V.release(); cnorm.release(); perm.release(); Q.release(); qnorm.release();
        qflags.release(); Qd.release(); mask.release(); keys.release(); keys_alt.release(); idx.release();
        idx_alt.release(); qkey.release(); tmp.release(); take.release(); out_index.release();
        samples.release(); cand_key.release(); cand_key_alt.release();
        cand_idx.release(); cand_idx_alt.release(); cnt.release(); seg_begin.release();
        seg_end.release(); blk_count.release();
        out_score.release();
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

// vector.rs:24-53, one query on the host. Returns its norm.
svl_status check_query(const float *q, int64_t len, int64_t index_dim, bool has_dim, int32_t which,
                       double &norm) {
    if (len <= 0)
        return fail(SVL_USAGE, "query %d: query embedding must have at least one dimension", which);
    if (len > MAX_EMBEDDING_DIMENSION)
        return fail(SVL_LIMIT, "query %d: query embedding has %lld dimensions, above the %lld-dimension cap",
                    which, (long long)len, (long long)MAX_EMBEDDING_DIMENSION);
    double sum = 0.0;
    for (int64_t d = 0; d < len; ++d) {
        if (!std::isfinite(q[d]))
            return fail(SVL_USAGE, "query %d: query embedding contains a non-finite value", which);
        sum += (double)q[d] * (double)q[d];
    }
    if (!std::isfinite(sum) || sum <= 0.0)
        return fail(SVL_USAGE,
                    "query %d: query embedding norm is zero or non-finite; cosine similarity is undefined",
                    which);
    norm = std::sqrt(sum);
    if (has_dim && len != index_dim)
        return fail(SVL_USAGE, "query %d: query embedding dimension %lld does not match the index dimension %lld",
                    which, (long long)len, (long long)index_dim);
    return SVL_OK;
}

// Pages much smaller than the index (offset + limit <= n / 16): exact top-K
// by threshold. S = 4096 evenly spaced keys per query are sorted; the sample
// at a rank with margin above the expected (offset + limit) / n quantile is a
// threshold, and every admitted key at or below it is a candidate (gathered
// in position order without atomics). When each
// query has at least min(offset + limit, admitted) candidates (and no more
// than the buffer holds), its page lies among them, and sorting only the
// candidates by (key, position) gives the ranking's exact entries; otherwise
// `selected` stays false and the full sort runs.
svl_status select_top(svl_vector_index *ix, int32_t nq, int64_t offset, int64_t limit,
                      const std::vector<int64_t> &take, const std::vector<int64_t> &pass,
                      int64_t *out_index, double *out_score, hipStream_t s, bool &selected) {
    selected = false;
    const int64_t n = ix->n, K = offset + limit;
    constexpr int S = SAMPLE_COUNT;
    if (n < 16 * S || K > n / 16) return SVL_OK;
    const int64_t stride = n / S;
    const double f = (double)K * S / (double)n;
    const int rank = (int)std::min<double>(S - 1, std::ceil(1.5 * f + 4.0 * std::sqrt(f) + 8.0));
    const int64_t cap = std::min<int64_t>(n, 2 * (int64_t)(rank + 1) * stride + 4096);
    if ((int64_t)nq * cap > (int64_t)UINT32_MAX) return SVL_OK;
    HIP_TRY(ix->samples.ensure((size_t)nq * S));
    HIP_TRY(ix->cand_key.ensure((size_t)(nq * cap)));
    HIP_TRY(ix->cand_key_alt.ensure((size_t)(nq * cap)));
    HIP_TRY(ix->cand_idx.ensure((size_t)(nq * cap)));
    HIP_TRY(ix->cand_idx_alt.ensure((size_t)(nq * cap)));
    HIP_TRY(ix->cnt.ensure((size_t)nq));
    HIP_TRY(ix->blk_count.ensure((size_t)nq * (size_t)candidate_blocks(n)));
    if (nq <= SELECT_SAMPLE_MAX_QUERIES)
        HIP_TRY(select_sample(ix->keys.p, nq, n, rank, ix->samples.p, s));
    else
        HIP_TRY(sort_samples(ix->keys.p, nq, n, ix->samples.p, s));
    HIP_TRY(launch_compact_keys(ix->keys.p, nq, n, ix->samples.p, S, rank, cap, ix->blk_count.p,
                                ix->cnt.p, ix->cand_key.p, ix->cand_idx.p, s));
    std::vector<unsigned int> cnt((size_t)nq);
    HIP_TRY(hipMemcpyAsync(cnt.data(), ix->cnt.p, (size_t)nq * sizeof(unsigned int),
                           hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    int64_t most = 0;
    for (int32_t q = 0; q < nq; ++q) {
        const int64_t need = std::min(K, pass[(size_t)q]);
        if ((int64_t)cnt[(size_t)q] < need || (int64_t)cnt[(size_t)q] > cap) return SVL_OK;
        most = std::max<int64_t>(most, cnt[(size_t)q]);
    }
    if (most <= CAND_LDS) {
        HIP_TRY(sort_candidates_lds(ix->cand_key.p, ix->cand_idx.p, ix->cand_key_alt.p,
                                    ix->cand_idx_alt.p, ix->cnt.p, nq, cap, most, s));
    } else {
        HIP_TRY(ix->seg_begin.ensure((size_t)nq));
        HIP_TRY(ix->seg_end.ensure((size_t)nq));
        size_t b = 0;
        HIP_TRY(sort_candidates(ix->cand_key.p, ix->cand_idx.p, ix->cand_key_alt.p,
                                ix->cand_idx_alt.p, ix->cnt.p, ix->seg_begin.p, ix->seg_end.p, nq,
                                cap, nullptr, &b, s));
        HIP_TRY(ix->tmp.ensure(std::max<size_t>(b, 1)));
        HIP_TRY(sort_candidates(ix->cand_key.p, ix->cand_idx.p, ix->cand_key_alt.p,
                                ix->cand_idx_alt.p, ix->cnt.p, ix->seg_begin.p, ix->seg_end.p, nq,
                                cap, ix->tmp.p, &b, s));
    }
    HIP_TRY(launch_gather_candidates(ix->cand_key_alt.p, ix->cand_idx_alt.p, nq, n, cap, ix->perm.p,
                                     offset, limit, ix->take.p, ix->out_index.p,
                                     ix->out_score.p, s));
    HIP_TRY(hipMemcpyAsync(out_index, ix->out_index.p, (size_t)(nq * limit) * 8,
                           hipMemcpyDeviceToHost, s));
    HIP_TRY(hipMemcpyAsync(out_score, ix->out_score.p, (size_t)(nq * limit) * 8,
                           hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    (void)take;
    selected = true;
    return SVL_OK;
}

// The ranking of `nq` validated queries already in ix->Q / ix->qnorm.
svl_status rank_loaded(svl_vector_index *ix, int32_t nq, const uint8_t *mask, int64_t mask_stride,
                       int64_t offset, int64_t limit, int64_t *out_index, double *out_score,
                       int64_t *out_count, hipStream_t s) {
    const int64_t n = ix->n;
    // admitted chunks per query, and the first admitted bad chunk (vector.rs:77-82)
    std::vector<int64_t> take((size_t)nq), pass((size_t)nq, n);
    for (int32_t q = 0; q < nq; ++q) {
        if (mask) {
            const uint8_t *m = mask + (int64_t)q * mask_stride;
            int64_t cnt = 0;
            for (int64_t c = 0; c < n; ++c) cnt += m[c] != 0;
            pass[(size_t)q] = cnt;
        }
        for (int64_t b : ix->bad_list)
            if (!mask || mask[(int64_t)q * mask_stride + b])
                return fail(SVL_INTERNAL, "query %d: chunk %llu has a zero or non-finite embedding norm",
                            q, (unsigned long long)ix->ids[(size_t)b]);
        take[(size_t)q] = std::max<int64_t>(0, std::min(limit, pass[(size_t)q] - offset));
        out_count[q] = take[(size_t)q];
    }
    if (n == 0 || limit == 0) return SVL_OK;
    const int64_t count = (int64_t)nq * n;
    if (count > (int64_t)UINT32_MAX) return fail(SVL_LIMIT, "queries x chunks exceeds 2^32 pairs");
    HIP_TRY(ix->keys.ensure((size_t)count));
    HIP_TRY(ix->keys_alt.ensure((size_t)count));
    HIP_TRY(ix->idx.ensure((size_t)count));
    HIP_TRY(ix->idx_alt.ensure((size_t)count));
    HIP_TRY(ix->qkey.ensure((size_t)count));
    HIP_TRY(ix->take.ensure((size_t)nq));
    HIP_TRY(ix->out_index.ensure((size_t)(nq * limit)));
    HIP_TRY(ix->out_score.ensure((size_t)(nq * limit)));
    const uint8_t *d_mask = nullptr;
    int64_t d_stride = 0;
    if (mask) {
        const int64_t rows = mask_stride == 0 ? 1 : nq;
        HIP_TRY(ix->mask.ensure((size_t)(rows * n)));
        for (int64_t r = 0; r < rows; ++r)
            HIP_TRY(hipMemcpyAsync(ix->mask.p + r * n, mask + r * mask_stride, (size_t)n,
                                   hipMemcpyHostToDevice, s));
        d_mask = ix->mask.p;
        d_stride = mask_stride == 0 ? 0 : n;
    }
    const int qb = cosine_query_block(nq);
    HIP_TRY(ix->Qd.ensure((size_t)(ix->D * ((nq + qb - 1) / qb * qb))));
    HIP_TRY(launch_cosine_keys(ix->V.p, ix->cnorm.p, ix->Q.p, ix->qnorm.p, nq, n, (int)ix->D,
                               d_mask, d_stride, ix->perm.p, ix->Qd.p, ix->keys.p, s));
    HIP_TRY(hipMemcpyAsync(ix->take.p, take.data(), (size_t)nq * 8, hipMemcpyHostToDevice, s));
    bool selected = false;
    ST_TRY(select_top(ix, nq, offset, limit, take, pass, out_index, out_score, s, selected));
    if (selected) return SVL_OK;
    size_t tmp_bytes = 0;
    const uint32_t *sorted = nullptr;
    HIP_TRY(rank_sort(ix->keys.p, ix->keys_alt.p, ix->idx.p, ix->idx_alt.p, ix->qkey.p, nq, n,
                      nullptr, &tmp_bytes, &sorted, s));
    HIP_TRY(ix->tmp.ensure(std::max<size_t>(tmp_bytes, 1)));
    HIP_TRY(rank_sort(ix->keys.p, ix->keys_alt.p, ix->idx.p, ix->idx_alt.p, ix->qkey.p, nq, n,
                      ix->tmp.p, &tmp_bytes, &sorted, s));
    HIP_TRY(launch_gather_hits(ix->keys.p, sorted, nq, n, ix->perm.p, offset, limit, ix->take.p,
                               ix->out_index.p, ix->out_score.p, s));
    HIP_TRY(hipMemcpyAsync(out_index, ix->out_index.p, (size_t)(nq * limit) * 8,
                           hipMemcpyDeviceToHost, s));
    HIP_TRY(hipMemcpyAsync(out_score, ix->out_score.p, (size_t)(nq * limit) * 8,
                           hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return SVL_OK;
}

svl_status check_page(int32_t nq, int64_t offset, int64_t limit, int64_t *out_index,
                      double *out_score, int64_t *out_count) {
    if (nq < 0 || offset < 0 || limit < 0) return fail(SVL_USAGE, "negative query count, offset or limit");
    if (nq > 0 && (!out_count || (limit > 0 && (!out_index || !out_score))))
        return fail(SVL_USAGE, "outputs are required");
    return SVL_OK;
}

}  // namespace

extern "C" {

svl_status svl_vector_index_create(svl_ctx *ctx, const float *embeddings,
                                   const uint64_t *chunk_ids, int64_t n, int64_t dimension,
                                   svl_vector_index **out) {
    if (!ctx || !out || n < 0 || (n > 0 && (!embeddings || !chunk_ids)))
        return fail(SVL_USAGE, "context, embeddings, chunk ids and output are required");
    *out = nullptr;
    if (n > 0 && (dimension <= 0 || dimension > MAX_EMBEDDING_DIMENSION))
        return fail(SVL_LIMIT, "embedding dimension %lld is outside 1..=%lld", (long long)dimension,
                    (long long)MAX_EMBEDDING_DIMENSION);
    if (n * std::max<int64_t>(dimension, 1) > MAX_TENSOR_ELEMENTS * 4)
        return fail(SVL_LIMIT, "index of %lld x %lld embeddings is too large", (long long)n,
                    (long long)dimension);
    std::unique_ptr<svl_vector_index> ix(new svl_vector_index());
    ix->device = ctx->device;
    ix->n = n;
    ix->D = n > 0 ? dimension : 0;
    HIP_TRY(hipSetDevice(ix->device));
    HIP_TRY(hipStreamCreateWithFlags(&ix->stream, hipStreamNonBlocking));
    ix->ids.assign(chunk_ids, chunk_ids + n);
    std::vector<int64_t> perm((size_t)n);
    std::iota(perm.begin(), perm.end(), 0);
    std::stable_sort(perm.begin(), perm.end(),
                     [&](int64_t a, int64_t b) { return chunk_ids[a] < chunk_ids[b]; });
    // squared sums in d order (vector.rs:71-78), chunk by chunk on host threads
    std::vector<double> norm((size_t)n);
    ix->bad.assign((size_t)n, 0);
    const int64_t D = ix->D;
    const int threads = (int)std::min<int64_t>(std::max(1u, std::thread::hardware_concurrency()),
                                               std::min<int64_t>(16, std::max<int64_t>(n / 1024, 1)));
    auto work = [&](int k) {
        for (int64_t c = k; c < n; c += threads) {
            const float *v = embeddings + c * D;
            double sum = 0.0;
            for (int64_t d = 0; d < D; ++d) sum += (double)v[d] * (double)v[d];
            if (!std::isfinite(sum) || sum <= 0.0) {
                ix->bad[(size_t)c] = 1;
                norm[(size_t)c] = 1.0;
            } else {
                norm[(size_t)c] = std::sqrt(sum);
            }
        }
    };
    std::vector<std::thread> pool;
    for (int k = 1; k < threads; ++k) pool.emplace_back(work, k);
    work(0);
    for (auto &t : pool) t.join();
    for (int64_t c = 0; c < n; ++c)
        if (ix->bad[(size_t)c]) ix->bad_list.push_back(c);
    if (n > 0) {
        std::vector<double> cn((size_t)n);
        for (int64_t p = 0; p < n; ++p) cn[(size_t)p] = norm[(size_t)perm[(size_t)p]];
        HIP_TRY(ix->V.ensure((size_t)(n * D)));
        HIP_TRY(ix->cnorm.ensure((size_t)n));
        HIP_TRY(ix->perm.ensure((size_t)n));
        // rows in chunk-id order, staged through a bounded host buffer
        const int64_t rows_per = std::max<int64_t>(1, ((int64_t)64 << 20) / (D * 4));
        std::vector<float> stage((size_t)(std::min(rows_per, n) * D));
        for (int64_t p0 = 0; p0 < n; p0 += rows_per) {
            const int64_t rows = std::min(rows_per, n - p0);
            for (int64_t r = 0; r < rows; ++r)
                std::copy(embeddings + perm[(size_t)(p0 + r)] * D,
                          embeddings + (perm[(size_t)(p0 + r)] + 1) * D, stage.data() + r * D);
            HIP_TRY(hipMemcpy(ix->V.p + p0 * D, stage.data(), (size_t)(rows * D) * 4,
                              hipMemcpyHostToDevice));
        }
        HIP_TRY(hipMemcpy(ix->cnorm.p, cn.data(), (size_t)n * 8, hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(ix->perm.p, perm.data(), (size_t)n * 8, hipMemcpyHostToDevice));
    }
    *out = ix.release();
    return SVL_OK;
}

svl_status svl_vector_index_destroy(svl_vector_index *index) {
    delete index;
    return SVL_OK;
}

int64_t svl_vector_index_size(const svl_vector_index *index) { return index ? index->n : -1; }

int64_t svl_vector_index_dimension(const svl_vector_index *index) {
    return index ? index->D : -1;
}

svl_status svl_vector_rank(svl_vector_index *ix, const float *queries, int32_t nq,
                           int64_t query_dim, const uint8_t *mask, int64_t mask_stride,
                           int64_t offset, int64_t limit, int64_t *out_index, double *out_score,
                           int64_t *out_count) {
    if (!ix || (nq > 0 && !queries)) return fail(SVL_USAGE, "index and queries are required");
    ST_TRY(check_page(nq, offset, limit, out_index, out_score, out_count));
    if (mask_stride != 0 && mask_stride < ix->n) return fail(SVL_USAGE, "mask stride is shorter than the index");
    std::lock_guard<std::mutex> lock(ix->mu);
    std::vector<double> qn((size_t)nq);
    for (int32_t q = 0; q < nq; ++q)
        ST_TRY(check_query(queries + (int64_t)q * std::max<int64_t>(query_dim, 0), query_dim, ix->D,
                           ix->n > 0, q, qn[(size_t)q]));
    if (nq == 0) return SVL_OK;
    HIP_TRY(hipSetDevice(ix->device));
    hipStream_t s = ix->stream;
    if (ix->n > 0) {
        HIP_TRY(ix->Q.ensure((size_t)(nq * ix->D)));
        HIP_TRY(ix->qnorm.ensure((size_t)nq));
        HIP_TRY(hipMemcpyAsync(ix->Q.p, queries, (size_t)(nq * ix->D) * 4, hipMemcpyHostToDevice, s));
        HIP_TRY(hipMemcpyAsync(ix->qnorm.p, qn.data(), (size_t)nq * 8, hipMemcpyHostToDevice, s));
    }
    return rank_loaded(ix, nq, mask, mask_stride, offset, limit, out_index, out_score, out_count, s);
}

svl_status svl_vector_rank_device(svl_vector_index *ix, const float *d_queries, int32_t nq,
                                  int64_t query_dim, const uint8_t *mask, int64_t mask_stride,
                                  int64_t offset, int64_t limit, int64_t *out_index,
                                  double *out_score, int64_t *out_count, void *stream) {
    if (!ix || (nq > 0 && !d_queries)) return fail(SVL_USAGE, "index and queries are required");
    ST_TRY(check_page(nq, offset, limit, out_index, out_score, out_count));
    if (mask_stride != 0 && mask_stride < ix->n) return fail(SVL_USAGE, "mask stride is shorter than the index");
    if (nq > 0 && query_dim <= 0)
        return fail(SVL_USAGE, "query embedding must have at least one dimension");
    if (query_dim > MAX_EMBEDDING_DIMENSION)
        return fail(SVL_LIMIT, "query embedding has %lld dimensions, above the %lld-dimension cap",
                    (long long)query_dim, (long long)MAX_EMBEDDING_DIMENSION);
    std::lock_guard<std::mutex> lock(ix->mu);
    if (nq == 0) return SVL_OK;
    HIP_TRY(hipSetDevice(ix->device));
    hipStream_t s = stream ? (hipStream_t)stream : ix->stream;
    HIP_TRY(ix->qnorm.ensure((size_t)nq));
    HIP_TRY(ix->qflags.ensure((size_t)nq));
    HIP_TRY(launch_query_norms(d_queries, nq, (int)query_dim, ix->qnorm.p, ix->qflags.p, s));
    std::vector<int> flags((size_t)nq);
    HIP_TRY(hipMemcpyAsync(flags.data(), ix->qflags.p, (size_t)nq * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    for (int32_t q = 0; q < nq; ++q) {
        if (flags[(size_t)q] & 1)
            return fail(SVL_USAGE, "query %d: query embedding contains a non-finite value", q);
        if (flags[(size_t)q] & 2)
            return fail(SVL_USAGE,
                        "query %d: query embedding norm is zero or non-finite; cosine similarity is undefined", q);
        if (ix->n > 0 && query_dim != ix->D)
            return fail(SVL_USAGE, "query %d: query embedding dimension %lld does not match the index dimension %lld",
                        q, (long long)query_dim, (long long)ix->D);
    }
    if (ix->n > 0) {
        HIP_TRY(ix->Q.ensure((size_t)(nq * ix->D)));
        HIP_TRY(hipMemcpyAsync(ix->Q.p, d_queries, (size_t)(nq * ix->D) * 4, hipMemcpyDeviceToDevice, s));
    }
    return rank_loaded(ix, nq, mask, mask_stride, offset, limit, out_index, out_score, out_count, s);
}

}  // extern "C"
