/*
 * CPU oracle, exact vector search: a C restatement of vector::rank
 * (src/index/vector.rs:17-97).
 *
 * TEST INFRASTRUCTURE ONLY: the oracle for the HIP cosine ranking, never part
 * of the product library. Built with -ffp-contract=off: the dot product and
 * the squared norms are accumulated in double in dimension order with a
 * separate multiply and add, as the reference does; the ranking is sorted by
 * f64::total_cmp descending, then ascending chunk id, then input order (the
 * reference's sort_by is stable).
 *
 * Parity pins (tests/test_oracle_search.py): the unit tests of
 * vector.rs:137-225 (scores 1, 1/sqrt(2), 0 and their order; filters; the
 * error kinds), scores against numpy's dot / norm in long double closed form,
 * and the order against Python's sorted() on (-score, chunk id, index).
 */
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "svl_oracle.h"

static int vs_fail(char *msg, size_t msg_len, int code, const char *fmt, ...) {
    if (msg && msg_len) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(msg, msg_len, fmt, ap);
        va_end(ap);
    }
    return code;
}

typedef struct {
    size_t index;
    double score;
    uint64_t id;
} vs_entry;

/* f64::total_cmp as an unsigned order */
static uint64_t total_key(double s) {
    uint64_t b;
    memcpy(&b, &s, 8);
    return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

static int vs_cmp(const void *pa, const void *pb) {
    const vs_entry *a = (const vs_entry *)pa, *b = (const vs_entry *)pb;
    const uint64_t ka = total_key(a->score), kb = total_key(b->score);
    if (ka != kb) return ka > kb ? -1 : 1; /* descending score */
    if (a->id != b->id) return a->id < b->id ? -1 : 1;
    return a->index < b->index ? -1 : (a->index > b->index);
}

int svlo_vector_rank(const float *query, size_t qlen, const float *emb, const uint64_t *ids,
                     size_t n, size_t dim, int has_dim, const unsigned char *mask,
                     size_t *out_index, double *out_score, size_t *out_count, char *msg,
                     size_t msg_len) {
    if (qlen == 0)
        return vs_fail(msg, msg_len, SVLO_USAGE, "query embedding must have at least one dimension");
    if (qlen > SVLO_MAX_EMBEDDING_DIMENSION)
        return vs_fail(msg, msg_len, SVLO_LIMIT, "query embedding has %zu dimensions", qlen);
    double query_sum = 0.0;
    for (size_t d = 0; d < qlen; ++d) {
        if (!isfinite(query[d]))
            return vs_fail(msg, msg_len, SVLO_USAGE, "query embedding contains a non-finite value");
        query_sum += (double)query[d] * (double)query[d];
    }
    if (!isfinite(query_sum) || query_sum <= 0.0)
        return vs_fail(msg, msg_len, SVLO_USAGE, "query embedding norm is zero or non-finite");
    const double query_norm = sqrt(query_sum);
    if (has_dim && qlen != dim)
        return vs_fail(msg, msg_len, SVLO_USAGE, "query dimension %zu does not match %zu", qlen, dim);
    vs_entry *scored = (vs_entry *)malloc(sizeof(vs_entry) * (n ? n : 1));
    if (!scored) return vs_fail(msg, msg_len, SVLO_INTERNAL, "out of memory");
    size_t m = 0;
    for (size_t c = 0; c < n; ++c) {
        if (mask && !mask[c]) continue;
        if (dim != qlen) {
            free(scored);
            return vs_fail(msg, msg_len, SVLO_INTERNAL, "chunk %llu has dimension %zu",
                           (unsigned long long)ids[c], dim);
        }
        const float *v = emb + c * dim;
        double dot = 0.0, vector_sum = 0.0;
        for (size_t d = 0; d < qlen; ++d) {
            const double q = (double)query[d], x = (double)v[d];
            dot += q * x;
            vector_sum += x * x;
        }
        if (!isfinite(vector_sum) || vector_sum <= 0.0) {
            free(scored);
            return vs_fail(msg, msg_len, SVLO_INTERNAL,
                           "chunk %llu has a zero or non-finite embedding norm",
                           (unsigned long long)ids[c]);
        }
        scored[m].index = c;
        scored[m].score = dot / (query_norm * sqrt(vector_sum));
        scored[m].id = ids[c];
        ++m;
    }
    qsort(scored, m, sizeof(vs_entry), vs_cmp);
    for (size_t i = 0; i < m; ++i) {
        out_index[i] = scored[i].index;
        out_score[i] = scored[i].score;
    }
    *out_count = m;
    free(scored);
    return SVLO_OK;
}
