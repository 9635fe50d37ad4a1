"""ctypes front-end of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
the cpu_baseline leg of bench.py, always as the checker.  The product library
never loads it.

Every function mirrors one reference routine; the C source names the Dart
file:line it restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

L2 = 0
IP = 1


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-C", _HERE, "-s", "-B", "liboracle.so"], check=True)


class _Range(ctypes.Structure):
    _fields_ = [
        ("nq", ctypes.c_int64),
        ("lims", ctypes.POINTER(ctypes.c_int64)),
        ("D", ctypes.POINTER(ctypes.c_float)),
        ("I", ctypes.POINTER(ctypes.c_int32)),
    ]


class _Pairs(ctypes.Structure):
    _fields_ = [
        ("npairs", ctypes.c_int64),
        ("i", ctypes.POINTER(ctypes.c_int32)),
        ("j", ctypes.POINTER(ctypes.c_int32)),
        ("s", ctypes.POINTER(ctypes.c_float)),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.orc_flat_search.argtypes = [p, i64, i64, p, i64, i64, ctypes.c_int, p, p, ctypes.c_int]
        L.orc_flat_search.restype = ctypes.c_int
        L.orc_flat_range_search.argtypes = [p, i64, i64, p, i64, ctypes.c_double, ctypes.c_int, ctypes.c_int]
        L.orc_flat_range_search.restype = ctypes.POINTER(_Range)
        L.orc_range_free.argtypes = [ctypes.POINTER(_Range)]
        L.orc_self_join.argtypes = [p, i64, i64, ctypes.c_double, i64, i64, ctypes.c_int]
        L.orc_self_join.restype = ctypes.POINTER(_Pairs)
        L.orc_pairs_free.argtypes = [ctypes.POINTER(_Pairs)]
        L.orc_kmeans_assign.argtypes = [p, i64, i64, p, i64, p, p, p, ctypes.c_int]
        L.orc_kmeans_assign.restype = ctypes.c_int
        L.orc_kmeans_update.argtypes = [p, i64, i64, p, i64, i64, p, p, p, i64]
        L.orc_kmeans_update.restype = ctypes.c_int64
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def flat_search(xb, xq, k: int, metric: int, nthreads: int = 1):
    """IndexFlat.search (index_flat.dart:62-97). Returns (D float32 nq x k, I int32 nq x k)."""
    xb = _f32(xb)
    xq = _f32(xq)
    n, d = xb.shape if xb.size else (0, xq.shape[1])
    nq = xq.shape[0]
    D = np.empty((nq, k), np.float32)
    I = np.empty((nq, k), np.int32)
    rc = lib().orc_flat_search(_ptr(xb), n, d, _ptr(xq), nq, k, metric, _ptr(D), _ptr(I), nthreads)
    if rc != 0:
        raise ValueError(f"orc_flat_search failed ({rc})")
    return D, I


class _Result:
    """The fields benchIndex reads of a SearchResult (index.dart:28-35)."""

    def __init__(self, D, I):
        self.distances, self.ids = D, I
        self.nq, self.k = D.shape


class FlatIndex:
    """The CPU IndexFlat (index_flat.dart:17-97) as an index object for the
    bench harness: the rows of the `IndexFlatL2` / `IndexFlatIP` rows of
    bench_faiss.dart:55-103, timed by the same benchIndex as the GPU index."""

    def __init__(self, xb, metric: int, nthreads: int = 1):
        self.xb = _f32(xb)
        self.metric, self.nthreads = int(metric), int(nthreads)

    @property
    def ntotal(self) -> int:
        return int(self.xb.shape[0])

    def search(self, xq, k: int):
        return _Result(*flat_search(self.xb, xq, k, self.metric, self.nthreads))


def flat_range_search(xb, xq, radius: float, metric: int, nthreads: int = 1):
    """IndexFlat.rangeSearch (index_flat.dart:99-137). Returns CSR (lims int64, D, I)."""
    xb = _f32(xb)
    xq = _f32(xq)
    n, d = xb.shape if xb.size else (0, xq.shape[1])
    nq = xq.shape[0]
    r = lib().orc_flat_range_search(_ptr(xb), n, d, _ptr(xq), nq, float(radius), metric, nthreads)
    if not r:
        raise ValueError("orc_flat_range_search failed")
    try:
        lims = np.ctypeslib.as_array(r.contents.lims, shape=(nq + 1,)).copy()
        tot = int(lims[-1])
        D = np.ctypeslib.as_array(r.contents.D, shape=(max(tot, 1),))[:tot].copy()
        I = np.ctypeslib.as_array(r.contents.I, shape=(max(tot, 1),))[:tot].copy()
    finally:
        lib().orc_range_free(r)
    return lims, D, I


def self_join(x, threshold: float, row_begin: int = 0, row_end: int | None = None, nthreads: int = 1):
    """Dedup pairs i<j with fp64 dot >= threshold (vector_dedup_demo.dart:115-128), sorted by (i, j)."""
    x = _f32(x)
    n, d = x.shape
    if row_end is None:
        row_end = n
    r = lib().orc_self_join(_ptr(x), n, d, float(threshold), row_begin, row_end, nthreads)
    if not r:
        raise ValueError("orc_self_join failed")
    try:
        m = int(r.contents.npairs)
        cnt = max(m, 1)
        i = np.ctypeslib.as_array(r.contents.i, shape=(cnt,))[:m].copy()
        j = np.ctypeslib.as_array(r.contents.j, shape=(cnt,))[:m].copy()
        s = np.ctypeslib.as_array(r.contents.s, shape=(cnt,))[:m].copy()
    finally:
        lib().orc_pairs_free(r)
    return i, j, s


def kmeans_assign(x, cen, nthreads: int = 1):
    """Kmeans assignment step (kmeans.dart:91-105). Returns (assign int32, best_sq float64, obj)."""
    x = _f32(x)
    cen = _f32(cen)
    n, d = x.shape
    K = cen.shape[0]
    assign = np.empty(n, np.int32)
    best = np.empty(n, np.float64)
    obj = ctypes.c_double(0.0)
    rc = lib().orc_kmeans_assign(_ptr(x), n, d, _ptr(cen), K, _ptr(assign), _ptr(best),
                                 ctypes.byref(obj), nthreads)
    if rc != 0:
        raise ValueError(f"orc_kmeans_assign failed ({rc})")
    return assign, best, obj.value


def kmeans_update(x, assign, cen, min_points: int = 1, jitter_u=None):
    """Kmeans update step (kmeans.dart:107-140). Returns (new centroids, counts, jitter used)."""
    x = _f32(x)
    n, d = x.shape
    cen = _f32(cen).copy()
    K = cen.shape[0]
    assign = np.ascontiguousarray(assign, dtype=np.int32)
    counts = np.empty(K, np.int32)
    ju = np.ascontiguousarray(jitter_u if jitter_u is not None else np.zeros(0), dtype=np.float64)
    used = lib().orc_kmeans_update(_ptr(x), n, d, _ptr(assign), K, min_points, _ptr(cen), _ptr(counts),
                                   _ptr(ju), ju.size)
    if used < 0:
        raise ValueError(f"orc_kmeans_update failed ({used})")
    return cen, counts, int(used)
