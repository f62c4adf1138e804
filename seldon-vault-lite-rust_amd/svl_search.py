"""Exact vector search on the MI355X backend, shaped like the reference crate's
index (src/index):

* ``VectorIndex`` — the vector view of ``Index::build`` (mod.rs:251-309):
  chunk embeddings resident in HBM
* ``VectorIndex.rank`` — ``vector::rank`` (vector.rs:17-97) for a batch of
  queries with per-query filters, sliced like ``Index::search``
  (mod.rs:347-359); ``rank_device`` takes queries already in HBM
* ``VectorIndex.search`` — the vector mode of ``Index::search`` with
  ``SearchRequest::validate`` (mod.rs:143-153) and one-based vector ranks

Scores are computed on the GPU in double exactly as the reference computes
them; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

import svl_amd
from svl_amd import SvlError, _check, lib

MAX_SEARCH_LIMIT = 1000          # index/mod.rs:21
MAX_SEARCH_OFFSET = 1_000_000    # index/mod.rs:23
MAX_EMBEDDING_DIMENSION = 8192   # storage/model.rs:35


def _load():
    L = lib()
    if not getattr(L, "_search_ready", False):
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        L.svl_vector_index_create.argtypes = [vp, vp, vp, i64, i64, ctypes.POINTER(vp)]
        L.svl_vector_index_destroy.argtypes = [vp]
        L.svl_vector_index_size.restype = i64
        L.svl_vector_index_size.argtypes = [vp]
        L.svl_vector_index_dimension.restype = i64
        L.svl_vector_index_dimension.argtypes = [vp]
        L.svl_vector_rank.argtypes = [vp, vp, i32, i64, vp, i64, i64, i64, vp, vp, vp]
        L.svl_vector_rank_device.argtypes = [vp, vp, i32, i64, vp, i64, i64, i64, vp, vp, vp, vp]
        L._search_ready = True
    return L


@dataclass
class VectorHit:
    """One ranked chunk (mod.rs:386-400 SearchHit, vector fields)."""
    index: int          # position in the indexed chunk list
    chunk_id: int
    score: float
    vector_rank: int    # one-based rank in the full ranking


class VectorIndex:
    def __init__(self, embeddings, chunk_ids, device: svl_amd.Device | None = None):
        self.device = device or svl_amd.Device.get(0)
        e = np.ascontiguousarray(embeddings, np.float32)
        if e.ndim != 2:
            e = e.reshape(len(chunk_ids), -1) if len(chunk_ids) else np.zeros((0, 0), np.float32)
        self.chunk_ids = np.ascontiguousarray(chunk_ids, np.uint64)
        if self.chunk_ids.size != e.shape[0]:
            raise SvlError(2, "one chunk id per embedding is required")
        h = ctypes.c_void_p()
        _check(_load().svl_vector_index_create(
            self.device.handle, ctypes.c_void_p(e.ctypes.data) if e.size else None,
            ctypes.c_void_p(self.chunk_ids.ctypes.data) if e.shape[0] else None, e.shape[0],
            e.shape[1], ctypes.byref(h)))
        self.handle = h

    def __del__(self):
        if getattr(self, "handle", None):
            _load().svl_vector_index_destroy(self.handle)
            self.handle = None

    def chunk_count(self):
        return int(_load().svl_vector_index_size(self.handle))

    def dimension(self):
        d = int(_load().svl_vector_index_dimension(self.handle))
        return None if self.chunk_count() == 0 else d

    def _mask(self, masks, nq):
        if masks is None:
            return None, 0, None
        m = np.ascontiguousarray(masks, np.uint8)
        if m.ndim == 1:
            return ctypes.c_void_p(m.ctypes.data), 0, m
        if m.shape[0] != nq:
            raise SvlError(2, "one mask row per query is required")
        return ctypes.c_void_p(m.ctypes.data), m.shape[1], m

    def _results(self, nq, limit, idx, score, count):
        return [(idx[q, : count[q]].copy(), score[q, : count[q]].copy()) for q in range(nq)]

    def rank(self, queries, masks=None, offset=0, limit=None):
        """[(indices, scores)] per query: ranking entries [offset, offset +
        limit) (limit None = the whole ranking)."""
        q = np.ascontiguousarray(queries, np.float32)
        if q.ndim == 1:
            q = q.reshape(1, -1)
        nq, dim = q.shape
        limit = self.chunk_count() if limit is None else int(limit)
        idx = np.zeros((max(nq, 1), max(limit, 1)), np.int64)
        score = np.zeros((max(nq, 1), max(limit, 1)), np.float64)
        count = np.zeros(max(nq, 1), np.int64)
        mp, stride, keep = self._mask(masks, nq)
        _check(_load().svl_vector_rank(self.handle, ctypes.c_void_p(q.ctypes.data), nq, dim, mp,
                                       stride, int(offset), limit,
                                       ctypes.c_void_p(idx.ctypes.data),
                                       ctypes.c_void_p(score.ctypes.data),
                                       ctypes.c_void_p(count.ctypes.data)))
        return self._results(nq, limit, idx, score, count)

    def rank_device(self, queries_dev_ptr: int, nq: int, dim: int, masks=None, offset=0,
                    limit=None, stream=None):
        limit = self.chunk_count() if limit is None else int(limit)
        idx = np.zeros((max(nq, 1), max(limit, 1)), np.int64)
        score = np.zeros((max(nq, 1), max(limit, 1)), np.float64)
        count = np.zeros(max(nq, 1), np.int64)
        mp, stride, keep = self._mask(masks, nq)
        _check(_load().svl_vector_rank_device(
            self.handle, ctypes.c_void_p(queries_dev_ptr), nq, dim, mp, stride, int(offset), limit,
            ctypes.c_void_p(idx.ctypes.data), ctypes.c_void_p(score.ctypes.data),
            ctypes.c_void_p(count.ctypes.data), ctypes.c_void_p(stream) if stream else None))
        return self._results(nq, limit, idx, score, count)

    def search(self, embedding, limit: int, offset: int = 0, mask=None):
        """Vector mode of Index::search (mod.rs:325-359)."""
        if limit == 0 or limit > MAX_SEARCH_LIMIT:
            raise SvlError(2, f"search limit must be between 1 and {MAX_SEARCH_LIMIT}")
        if offset > MAX_SEARCH_OFFSET:
            raise SvlError(2, f"search offset must not exceed {MAX_SEARCH_OFFSET}")
        idx, score = self.rank(embedding, None if mask is None else np.asarray(mask)[None],
                               offset, limit)[0]
        return [VectorHit(int(i), int(self.chunk_ids[i]), float(s), offset + k + 1)
                for k, (i, s) in enumerate(zip(idx, score))]
