"""Result containers and the Index contract (lib/core/vector_store/index.dart).

Python mirror of the reference's Dart types on the flat-search path:
Metric (index.dart:16), SearchResult (:28-35), RangeSearchResult (:49-99) and
the abstract Index (:123-179).  Rows are numpy arrays: distances float32,
ids int32, as the reference's Float32List / Int32List.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass

import numpy as np


class Metric(enum.IntEnum):
    """index.dart:16.  Values are the FAISDART codes (index_io.dart:233): 0 = L2, 1 = IP."""

    l2 = 0
    innerProduct = 1


@dataclass
class SearchResult:
    """index.dart:28-35: distances[i][j] / ids[i][j] of query i's j-th neighbour.

    Missing slots hold +inf (L2) / -inf (IP) with id -1."""

    distances: np.ndarray  # (nq, k) float32
    ids: np.ndarray  # (nq, k) int32

    @property
    def nq(self) -> int:
        return int(self.distances.shape[0])

    @property
    def k(self) -> int:
        return 0 if self.nq == 0 else int(self.distances.shape[1])


@dataclass
class RangeSearchResult:
    """index.dart:49-99: CSR layout; query qi's hits are [limits[qi], limits[qi+1])."""

    limits: np.ndarray  # (nq + 1,) int32 in the reference; int64 here (no 2^31 cap on hits)
    distances: np.ndarray  # float32
    ids: np.ndarray  # int32

    @property
    def nq(self) -> int:
        return int(self.limits.shape[0]) - 1

    @property
    def total_matches(self) -> int:
        return 0 if self.limits.size == 0 else int(self.limits[-1])

    def length_for(self, qi: int) -> int:
        return int(self.limits[qi + 1] - self.limits[qi])

    def to_rows(self):
        """index.dart:88-98: per-query (distances, ids) views."""
        ds = [self.distances[self.limits[q]:self.limits[q + 1]] for q in range(self.nq)]
        ids = [self.ids[self.limits[q]:self.limits[q + 1]] for q in range(self.nq)]
        return ds, ids


def as_rows(xs, d: int) -> np.ndarray:
    """Accepts a (n, d) array or a list of length-d rows (the reference's
    List<Float32List>); raises ValueError on a length mismatch like
    index_flat.dart:40-44 / :70-72."""
    if isinstance(xs, np.ndarray):
        a = xs
    else:
        rows = list(xs)
        for i, r in enumerate(rows):
            if len(r) != d:
                raise ValueError(f"vector {i} has length {len(r)}, expected {d}")
        a = np.asarray(rows, dtype=np.float32) if rows else np.zeros((0, d), np.float32)
    if a.ndim != 2 or (a.shape[0] > 0 and a.shape[1] != d):
        raise ValueError(f"expected rows of length {d}, got shape {a.shape}")
    return a


def recall_at_k(result: SearchResult, truth: SearchResult, k: int) -> float:
    """bench.dart:356-371: |result ∩ truth| / (nq * k), truth ids of -1 ignored."""
    hit = 0
    total = 0
    for qi in range(result.nq):
        gold = {int(i) for i in truth.ids[qi, :k] if i >= 0}
        hit += sum(1 for j in range(k) if int(result.ids[qi, j]) in gold)
        total += k
    return 0.0 if total == 0 else hit / total


class Index:
    """index.dart:123-179.  Subclasses set d/metric and implement add/search."""

    def __init__(self, d: int, metric: Metric):
        self.d = int(d)
        self.metric = Metric(metric)
        self.is_trained = True

    @property
    def ntotal(self) -> int:  # pragma: no cover - overridden
        raise NotImplementedError

    def train(self, xs) -> None:
        self.is_trained = True

    def add(self, xs) -> None:  # pragma: no cover - abstract
        raise NotImplementedError

    def search(self, queries, k: int) -> SearchResult:  # pragma: no cover - abstract
        raise NotImplementedError

    def range_search(self, queries, radius: float) -> RangeSearchResult:
        raise NotImplementedError(f"{type(self).__name__} does not support rangeSearch")

    def remove_ids(self, ids) -> int:
        raise NotImplementedError(f"{type(self).__name__} does not support removeIds")

    # Dart-style aliases of the reference's method names
    def rangeSearch(self, queries, radius: float) -> RangeSearchResult:
        return self.range_search(queries, radius)

    def removeIds(self, ids) -> int:
        return self.remove_ids(ids)

    def addRows(self, xs) -> None:
        self.add(as_rows(xs, self.d))

    def searchRows(self, queries, k: int) -> SearchResult:
        return self.search(as_rows(queries, self.d), k)
