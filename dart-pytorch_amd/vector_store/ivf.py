"""IndexIVFFlat's coarse path on the GPU flat scan
(lib/core/vector_store/index_ivf_flat.dart).

- train (:84-95): Kmeans(d, nlist, niter=kmeansIters, seed).train on the
  GPU (k-means++ init, vs_kmeans_step iterations); the centroids go into
  the coarse quantizer, a GpuIndexFlat of the index's metric;
- add (:98-130): each vector's cell is quantizer.search(xs, 1) (the fused
  k = 1 search); the vectors are stored in HBM in insertion order (ids
  continue from ntotal) and their ids appended to the cell's list;
- search (:132-171): quantizer.search(queries, nprobe) picks the cells, and
  the fine scan over the probed lists runs on the GPU too
  (vs_index_search_subsets: fp64 scores in dimension order, the k best per
  query by (fp32 score, id), sentinels when fewer vectors were probed).

The probes' order and the lists' insertion order do not change the result
except inside exact ties (the reference's TopK keeps whichever tied row its
heap history left; here the lowest id).
"""
from __future__ import annotations

import numpy as np

from .gpu_index_flat import GpuIndexFlat
from .index import Index, Metric, SearchResult, as_rows
from .kmeans import Kmeans


class IndexIVFFlat(Index):
    """index_ivf_flat.dart:16-26: IndexIVFFlat(d, nlist, metric=l2, nprobe=1,
    kmeansIters=20, seed=1234)."""

    def __init__(self, d: int, nlist: int, metric: Metric = Metric.l2, nprobe: int = 1,
                 kmeans_iters: int = 20, seed: int = 1234, device: int = 0):
        super().__init__(d, metric)
        self.nlist, self.nprobe = int(nlist), int(nprobe)
        self.kmeans_iters, self.seed, self.device = int(kmeans_iters), int(seed), device
        self.quantizer = GpuIndexFlat(d, self.metric, storage="f32", device=device)
        self._store = GpuIndexFlat(d, self.metric, storage="f32", device=device)
        self.is_trained = False
        self._lists = [[] for _ in range(self.nlist)]

    @property
    def ntotal(self) -> int:
        return self._store.ntotal

    @property
    def inv_lists(self):
        """invLists (index_ivf_flat.dart:52-55): ids per cell, insertion order."""
        return self._lists

    def close(self) -> None:
        self.quantizer.close()
        self._store.close()

    def train(self, xs) -> None:
        x = as_rows(xs, self.d) if not isinstance(xs, np.ndarray) else np.asarray(xs, np.float32)
        if x.shape[0] < self.nlist:
            raise ValueError(f"IndexIVFFlat.train: need >= nlist={self.nlist} vectors, "
                             f"got {x.shape[0]}")
        res = Kmeans(self.d, self.nlist, niter=self.kmeans_iters, seed=self.seed,
                     device=self.device).train(x)
        self.quantizer.add(res.centroids)
        self.is_trained = True

    def add(self, xs) -> None:
        if not self.is_trained:
            raise RuntimeError("IndexIVFFlat.add called before train()")
        x = as_rows(xs, self.d) if not isinstance(xs, np.ndarray) else np.asarray(xs, np.float32)
        if x.shape[0] == 0:
            return
        cells = self.quantizer.search(x, 1).ids[:, 0]
        base = self.ntotal
        self._store.add(x)
        for i, c in enumerate(cells.tolist()):
            self._lists[c].append(base + i)

    def search(self, queries, k: int) -> SearchResult:
        if not self.is_trained:
            raise RuntimeError("IndexIVFFlat.search before train()")
        q = as_rows(queries, self.d) if not isinstance(queries, np.ndarray) else np.asarray(queries, np.float32)
        nq = q.shape[0]
        if nq == 0:
            return SearchResult(np.zeros((0, k), np.float32), np.zeros((0, k), np.int32))
        probes = self.quantizer.search(q, self.nprobe).ids  # (nq, nprobe), -1 past nlist
        sizes = np.array([len(l) for l in self._lists], np.int64)
        starts = np.zeros(self.nlist + 1, np.int64)
        np.cumsum(sizes, out=starts[1:])
        ids = np.fromiter((i for l in self._lists for i in l), np.int32, count=int(starts[-1]))
        valid = probes >= 0
        cell = np.where(valid, probes, 0)
        seg_off = np.where(valid, starts[cell], 0)
        seg_len = np.where(valid, sizes[cell], 0)
        return self._store.search_subsets(q, k, ids, seg_off, seg_len)
