"""Pins of the vector-search oracle (oracle/svl_oracle_search.c, a restatement
of vector::rank, src/index/vector.rs:17-97): the unit tests of
vector.rs:137-225, scores against an exact long-double closed form, and the
order against Python's sorted() on (-score, chunk id, input index)."""
import math

import numpy as np
import pytest

from oracle import oracle as O


def test_ranks_by_cosine_similarity():
    # vector.rs:139-156
    idx, score = O.vector_rank([1.0, 0.0], [[1.0, 0.0], [0.0, 1.0], [1.0, 1.0]], [1, 2, 3])
    assert list(idx) == [0, 2, 1]
    assert abs(score[0] - 1.0) < 1e-9 and abs(score[1] - math.sqrt(0.5)) < 1e-6
    assert abs(score[2]) < 1e-9


def test_filters_exclude_chunks():
    # vector.rs:158-177
    idx, _ = O.vector_rank([1.0, 0.0], [[1.0, 0.0], [1.0, 0.0]], [1, 2], mask=[0, 1])
    assert list(idx) == [1]


@pytest.mark.parametrize("query,status", [
    ([1.0, 0.0, 0.0], 2),            # dimension mismatch (vector.rs:179-188)
    ([0.0, 0.0], 2), ([np.nan, 1.0], 2), ([np.inf, 0.0], 2),   # :190-200
    ([], 2),
    ([1.0] * 8193, 5),
])
def test_query_errors(query, status):
    with pytest.raises(O.OracleError) as e:
        O.vector_rank(query, [[1.0, 0.0]], [1])
    assert e.value.status == status


def test_empty_index_and_bad_chunks():
    # vector.rs:202-206
    idx, score = O.vector_rank([1.0, 0.0], np.zeros((0, 2), np.float32), [])
    assert idx.size == 0
    with pytest.raises(O.OracleError) as e:       # zero-norm chunk admitted
        O.vector_rank([1.0, 0.0], [[1.0, 0.0], [0.0, 0.0]], [1, 2])
    assert e.value.status == 7
    idx, _ = O.vector_rank([1.0, 0.0], [[1.0, 0.0], [0.0, 0.0]], [1, 2], mask=[1, 0])
    assert list(idx) == [0]                       # filtered out: no error


def test_scores_and_order_against_closed_form():
    rng = np.random.default_rng(3)
    n, d = 300, 48
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb[50:60] = emb[10]                          # exact ties
    emb[60] = -emb[10]
    ids = rng.permutation(np.arange(1, n + 1) * 7).astype(np.uint64)
    q = rng.standard_normal(d).astype(np.float32)
    idx, score = O.vector_rank(q, emb, ids)
    exact = [float(np.longdouble(np.dot(q.astype(np.longdouble), emb[i].astype(np.longdouble))) /
                   (np.sqrt(np.dot(q.astype(np.longdouble), q.astype(np.longdouble))) *
                    np.sqrt(np.dot(emb[i].astype(np.longdouble), emb[i].astype(np.longdouble)))))
             for i in range(n)]
    for i, s in zip(idx, score):
        assert abs(s - exact[i]) <= 1e-12
    want = sorted(range(n), key=lambda i: (-score[list(idx).index(i)], int(ids[i]), i))
    assert list(idx) == want
    tie = [i for i in idx if 50 <= i < 60 or i == 10]
    assert [int(ids[i]) for i in tie] == sorted(int(ids[i]) for i in tie)
