"""Wrapper indexes of the vector store over the GPU flat index: the
reference's IndexIDMap (index_id_map.dart), IndexPreTransform with
L2NormTransform (index_pre_transform.dart, l2_norm_transform.dart),
IndexRefineFlat (index_refine_flat.dart) and IndexShards
(index_shards.dart), with the reference's semantics:

- IndexIDMap: add assigns sequential external ids, addWithIds takes them
  (int32 range); search / rangeSearch rewrite internal ids to external ones,
  -1 slots untouched; removeIds takes external ids and compacts the table;
- IndexPreTransform: every vector and query passes the transform chain
  before the inner index (the chain's dIn / dOut must line up);
- IndexRefineFlat: search pulls min(k * kFactor, max(ntotal, 1)) candidates
  from the base index and re-ranks them exactly against the refine store --
  on the GPU: the candidates are each query's row subset of
  vs_index_search_subsets over the fp32 refine store;
- IndexShards: add deals vectors round-robin by external id (id % nshards);
  search asks every shard for k and keeps the k best of the union by the
  shards' fp32 scores, external id = local id * nshards + shard.

Ties are ordered by id here; the reference's TopK leaves them in heap order.
"""
from __future__ import annotations

import numpy as np

from .gpu_index_flat import GpuIndexFlat
from .index import Index, Metric, RangeSearchResult, SearchResult, as_rows

INT32_MIN, INT32_MAX = -(1 << 31), (1 << 31) - 1


def _rows(xs, d):
    return np.asarray(xs, np.float32) if isinstance(xs, np.ndarray) else as_rows(xs, d)


class L2NormTransform:
    """l2_norm_transform.dart:17-46: o = v / sqrt(fp64 sum of v*v in
    dimension order), rounded to fp32; zero rows stay zero."""

    def __init__(self, d: int):
        self.d_in = self.d_out = int(d)
        self.is_trained = True

    def apply(self, xs) -> np.ndarray:
        x = _rows(xs, self.d_in)
        if x.ndim != 2 or (x.shape[0] and x.shape[1] != self.d_in):
            raise ValueError(f"expected rows of length {self.d_in}, got shape {x.shape}")
        x64 = x.astype(np.float64)
        s = np.cumsum(x64 * x64, axis=1)[:, -1] if x.shape[0] else np.zeros(0)
        norm = np.sqrt(s)
        inv = np.divide(1.0, norm, out=np.zeros_like(norm), where=norm > 0)
        return (x64 * inv[:, None]).astype(np.float32)


class IndexIDMap(Index):
    """index_id_map.dart:14-150."""

    def __init__(self, inner: Index):
        super().__init__(inner.d, inner.metric)
        self.inner = inner
        self.is_trained = inner.is_trained
        self._ext: list[int] = []

    @property
    def ntotal(self) -> int:
        return len(self._ext)

    def train(self, xs) -> None:
        self.inner.train(xs)
        self.is_trained = self.inner.is_trained

    def add(self, xs) -> None:
        x = _rows(xs, self.d)
        start = len(self._ext)
        self.add_with_ids(x, list(range(start, start + x.shape[0])))

    def add_with_ids(self, xs, ids) -> None:
        x = _rows(xs, self.d)
        ids = [int(i) for i in ids]
        if x.shape[0] != len(ids):
            raise ValueError(f"addWithIds: xs ({x.shape[0]}) and ids ({len(ids)}) length mismatch")
        for i, v in enumerate(ids):
            if v < INT32_MIN or v > INT32_MAX:
                raise ValueError(f"addWithIds: id {v} at position {i} does not fit in int32")
        self.inner.add(x)
        self._ext.extend(ids)

    addWithIds = add_with_ids

    def id_of(self, i: int) -> int:
        return self._ext[i]

    def internal_of(self, ext: int) -> int:
        # the reference's reverse map is built by one pass in offset order,
        # so a duplicated external id maps to its last offset
        # (index_id_map.dart internalOf)
        for i in range(len(self._ext) - 1, -1, -1):
            if self._ext[i] == ext:
                return i
        return -1

    def _map(self, ids: np.ndarray) -> np.ndarray:
        ext = np.asarray(self._ext, np.int64)
        ok = (ids >= 0) & (ids < len(ext))
        out = ids.astype(np.int64).copy()
        out[ok] = ext[ids[ok]]
        return out.astype(np.int32)

    def search(self, queries, k: int) -> SearchResult:
        r = self.inner.search(queries, k)
        return SearchResult(r.distances, self._map(r.ids))

    def range_search(self, queries, radius: float) -> RangeSearchResult:
        r = self.inner.range_search(queries, radius)
        return RangeSearchResult(r.limits, r.distances, self._map(r.ids))

    def remove_ids(self, ids) -> int:
        rev = {e: i for i, e in enumerate(self._ext)}
        internal = {rev[e] for e in ids if e in rev}
        if not internal:
            return 0
        removed = self.inner.remove_ids(internal)
        self._ext = [e for i, e in enumerate(self._ext) if i not in internal]
        return removed


class IndexPreTransform(Index):
    """index_pre_transform.dart:16-110."""

    def __init__(self, chain, inner: Index):
        chain = list(chain)
        super().__init__(chain[0].d_in if chain else inner.d, inner.metric)
        expected = self.d
        for i, tr in enumerate(chain):
            if tr.d_in != expected:
                raise ValueError(f"IndexPreTransform: chain[{i}].dIn={tr.d_in} expected {expected}")
            expected = tr.d_out
        if expected != inner.d:
            raise ValueError(f"IndexPreTransform: chain outputs dim {expected} but inner.d={inner.d}")
        self.chain, self.inner = chain, inner
        self.is_trained = inner.is_trained and all(t.is_trained for t in chain)

    @property
    def ntotal(self) -> int:
        return self.inner.ntotal

    def _forward(self, xs) -> np.ndarray:
        cur = _rows(xs, self.d)
        for tr in self.chain:
            cur = tr.apply(cur)
        return cur

    def train(self, xs) -> None:
        self.inner.train(self._forward(xs))
        self.is_trained = self.inner.is_trained and all(t.is_trained for t in self.chain)

    def add(self, xs) -> None:
        if not self.is_trained:
            self.train(xs)
        self.inner.add(self._forward(xs))

    def search(self, queries, k: int) -> SearchResult:
        return self.inner.search(self._forward(queries), k)

    def range_search(self, queries, radius: float) -> RangeSearchResult:
        return self.inner.range_search(self._forward(queries), radius)

    def remove_ids(self, ids) -> int:
        return self.inner.remove_ids(ids)


class IndexRefineFlat(Index):
    """index_refine_flat.dart:26-91, the exact re-rank on the GPU."""

    def __init__(self, base: Index, k_factor: int = 4, device: int = 0):
        super().__init__(base.d, base.metric)
        self.base, self.k_factor = base, int(k_factor)
        self.refine = GpuIndexFlat(base.d, base.metric, storage="f32", device=device)
        self.is_trained = base.is_trained

    @property
    def ntotal(self) -> int:
        return self.refine.ntotal

    def close(self) -> None:
        self.refine.close()

    def train(self, xs) -> None:
        self.base.train(xs)
        self.is_trained = self.base.is_trained

    def add(self, xs) -> None:
        if not self.is_trained:
            raise RuntimeError("IndexRefineFlat.add before train()")
        x = _rows(xs, self.d)
        self.base.add(x)
        self.refine.add(x)

    def search(self, queries, k: int) -> SearchResult:
        if not self.is_trained:
            raise RuntimeError("IndexRefineFlat.search before train()")
        q = _rows(queries, self.d)
        nq = q.shape[0]
        if nq == 0:
            return SearchResult(np.zeros((0, k), np.float32), np.zeros((0, k), np.int32))
        coarse_k = min(k * self.k_factor, max(self.ntotal, 1))
        cand = self.base.search(q, coarse_k).ids
        valid = cand >= 0
        lens = valid.sum(axis=1).astype(np.int64)
        offs = np.zeros(nq, np.int64)
        np.cumsum(lens[:-1], out=offs[1:])
        ids = cand[valid].astype(np.int32)  # row-major: each query's valid candidates in order
        return self.refine.search_subsets(q, k, ids, offs[:, None], lens[:, None])


class IndexShards(Index):
    """index_shards.dart:14-120 (shards searched one after the other)."""

    def __init__(self, shards):
        shards = list(shards)
        if not shards:
            raise ValueError("IndexShards: need at least one shard")
        super().__init__(shards[0].d, shards[0].metric)
        for s in shards:
            if s.d != self.d or s.metric != self.metric:
                raise ValueError("IndexShards: shards must share d and metric")
        self.shards = shards
        # shards that already hold rows count from the start, as the
        # reference's constructor folds their ntotal
        self._ntotal = sum(int(s.ntotal) for s in shards)
        self.is_trained = all(s.is_trained for s in shards)

    @property
    def nshards(self) -> int:
        return len(self.shards)

    @property
    def ntotal(self) -> int:
        return self._ntotal

    def train(self, xs) -> None:
        for s in self.shards:
            if not s.is_trained:
                s.train(xs)
        self.is_trained = all(s.is_trained for s in self.shards)

    def add(self, xs) -> None:
        x = _rows(xs, self.d)
        if x.shape[0] == 0:
            return
        ext = self._ntotal + np.arange(x.shape[0])
        for s in range(self.nshards):
            part = x[ext % self.nshards == s]
            if part.shape[0]:
                self.shards[s].add(part)
        self._ntotal += x.shape[0]

    def search(self, queries, k: int) -> SearchResult:
        q = _rows(queries, self.d)
        nq = q.shape[0]
        Ds, Is = [], []
        for s, sh in enumerate(self.shards):
            r = sh.search(q, k)
            Ds.append(r.distances)
            Is.append(np.where(r.ids >= 0, r.ids.astype(np.int64) * self.nshards + s, -1))
        D = np.concatenate(Ds, axis=1) if Ds else np.zeros((nq, 0), np.float32)
        I = np.concatenate(Is, axis=1) if Is else np.zeros((nq, 0), np.int64)
        sgn = 1.0 if self.metric == Metric.l2 else -1.0
        outD = np.full((nq, k), np.inf if sgn > 0 else -np.inf, np.float32)
        outI = np.full((nq, k), -1, np.int32)
        for qi in range(nq):
            ok = I[qi] >= 0
            d, i = D[qi][ok], I[qi][ok]
            order = np.lexsort((i, sgn * d.astype(np.float64)))[:k]
            outD[qi, :len(order)] = d[order]
            outI[qi, :len(order)] = i[order]
        return SearchResult(outD, outI)
