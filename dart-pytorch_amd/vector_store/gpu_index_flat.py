"""GpuIndexFlat on MI355X: the drop-in for lib/core/vector_store/gpu_index_flat.dart.

The reference class (gpu_index_flat.dart:40-194) keeps a CPU IndexFlat and on
every search re-uploads, transposes and multiplies the whole database, copies
the nq x ntotal score matrix back and selects top-k in Dart.  Here the
vectors live in HBM for the index's lifetime and one library call returns the
k best per query; rangeSearch and removeIds, which the reference GPU class
does not override (they throw), are supported.

Constructors and members follow the reference: GpuIndexFlat.l2(d),
GpuIndexFlat.ip(d), GpuIndexFlat.wrap(flat), warmup(), ntotal, d, metric,
is_trained, add/search/range_search/remove_ids/reconstruct.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _native as N
from .index import Index, Metric, RangeSearchResult, SearchResult, as_rows


def _dtype_code(a: np.ndarray) -> tuple[np.ndarray, int]:
    """float32 rows, or bfloat16 rows passed as uint16 bit patterns."""
    if a.dtype == np.uint16:
        return np.ascontiguousarray(a), N.VS_DTYPE_BF16
    return np.ascontiguousarray(a, dtype=np.float32), N.VS_DTYPE_F32


# Planner options applied to every index this module creates or adopts
# (vs_index_set_option; the library's defaults when empty).  Test support:
# tests reach every kernel variant on small inputs by forcing a path here.
DEFAULT_OPTIONS: dict[str, int] = {}


class GpuIndexFlat(Index):
    """Exact flat index whose vectors stay resident on one GPU.

    storage: "f32" (the reference's Float32List), "bf16" (rounded once at
    add), or "auto" (bf16 while every value is exactly a bf16 value, which
    gives fp32 results at half the HBM traffic; fp32 otherwise)."""

    _STORAGE = {"f32": N.VS_STORAGE_F32, "bf16": N.VS_STORAGE_BF16, "auto": N.VS_STORAGE_AUTO}

    def __init__(self, d: int, metric: Metric = Metric.l2, storage: str = "auto", device: int = 0):
        super().__init__(d, metric)
        if d <= 0:
            raise ValueError(f"d must be > 0, got {d}")
        self._lib = N.load()
        self.device = device
        h = ctypes.c_void_p()
        N.check(self._lib.vs_index_create(device, int(d), int(self.metric), self._STORAGE[storage],
                                          ctypes.byref(h)))
        self._h = h
        self._apply_default_options()

    def _apply_default_options(self) -> None:
        for name, value in DEFAULT_OPTIONS.items():
            self.set_option(name, value)

    def set_option(self, name: str, value: int) -> None:
        """Force a planner option of this index (vs_index_set_option)."""
        N.check(self._lib.vs_index_set_option(self._h, name.encode(), int(value)))

    # --- constructors (gpu_index_flat.dart:46-57) ---
    @classmethod
    def l2(cls, d: int, **kw) -> "GpuIndexFlat":
        return cls(d, Metric.l2, **kw)

    @classmethod
    def ip(cls, d: int, **kw) -> "GpuIndexFlat":
        return cls(d, Metric.innerProduct, **kw)

    @classmethod
    def _adopt(cls, handle, device: int = 0) -> "GpuIndexFlat":
        """Wrap an index handle the library created (e.g. vs_index_load_flat)."""
        lib = N.load()
        g = cls.__new__(cls)
        Index.__init__(g, int(lib.vs_index_d(handle)), Metric(lib.vs_index_metric(handle)))
        g._lib = lib
        g.device = device
        g._h = handle
        g._apply_default_options()
        return g

    @classmethod
    def load(cls, src, storage: str = "auto", device: int = 0) -> "GpuIndexFlat":
        """readIndex / readFaissIndex of a flat index straight into HBM."""
        from .io import load_flat

        return load_flat(src, storage=storage, device=device)

    @classmethod
    def wrap(cls, src, **kw) -> "GpuIndexFlat":
        """Adopt an existing flat index (anything with d, metric, ntotal and
        reconstruct_n), copying its vectors to the GPU once."""
        g = cls(src.d, Metric(src.metric), **kw)
        n = int(src.ntotal)
        if n:
            g.add(src.reconstruct_n(0, n))
        return g

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.vs_index_destroy(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    @property
    def ntotal(self) -> int:
        return int(self._lib.vs_index_ntotal(self._h))

    @property
    def storage(self) -> str:
        return "bf16" if self._lib.vs_index_storage(self._h) == 1 else "f32"

    def warmup(self) -> None:
        """Vectors are resident from add(); kept for API parity (gpu_index_flat.dart:89)."""
        N.check(self._lib.vs_index_sync(self._h))

    def reserve(self, n: int) -> None:
        N.check(self._lib.vs_index_reserve(self._h, int(n)))

    def reset(self) -> None:
        N.check(self._lib.vs_index_reset(self._h))

    # --- data in ---
    def add(self, xs) -> None:
        """index_flat.dart:23-51: ids continue from ntotal."""
        a, code = _dtype_code(as_rows(xs, self.d) if not isinstance(xs, np.ndarray) else xs)
        if a.ndim != 2 or a.shape[1] != self.d:
            if a.size == 0:
                return
            raise ValueError(f"expected rows of length {self.d}, got shape {a.shape}")
        if a.shape[0] == 0:
            return
        N.check(self._lib.vs_index_add(self._h, a.ctypes.data_as(ctypes.c_void_p), code, a.shape[0]))

    def add_device(self, buf: N.DeviceBuffer, n: int, dtype: int = N.VS_DTYPE_F32) -> None:
        N.check(self._lib.vs_index_add_device(self._h, buf.ptr, dtype, int(n)))

    def reconstruct(self, i: int) -> np.ndarray:
        """index_flat.dart:55-60 (RangeError -> ValueError)."""
        return self.reconstruct_n(i, 1)[0]

    def reconstruct_n(self, i0: int, n: int) -> np.ndarray:
        out = np.empty((int(n), self.d), np.float32)
        N.check(self._lib.vs_index_reconstruct(self._h, int(i0), int(n),
                                               out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def remove_ids(self, ids) -> int:
        """index_flat.dart:139-160: compact, renumber from 0, return the count removed."""
        arr = np.fromiter((int(i) for i in ids), dtype=np.int64)
        removed = ctypes.c_int64(0)
        N.check(self._lib.vs_index_remove_ids(self._h, arr.ctypes.data_as(ctypes.c_void_p), arr.size,
                                              ctypes.byref(removed)))
        return int(removed.value)

    # --- search ---
    def search(self, queries, k: int) -> SearchResult:
        """index_flat.dart:62-97 / gpu_index_flat.dart:119-193."""
        q, code = _dtype_code(queries if isinstance(queries, np.ndarray) else as_rows(queries, self.d))
        nq = q.shape[0] if q.ndim == 2 else 0
        if nq == 0:
            return SearchResult(np.zeros((0, k), np.float32), np.zeros((0, k), np.int32))
        if q.shape[1] != self.d:
            raise ValueError(f"query length {q.shape[1]} != {self.d}")
        D = np.empty((nq, k), np.float32)
        I = np.empty((nq, k), np.int32)
        N.check(self._lib.vs_index_search(self._h, q.ctypes.data_as(ctypes.c_void_p), code, nq, int(k),
                                          D.ctypes.data_as(ctypes.c_void_p),
                                          I.ctypes.data_as(ctypes.c_void_p)))
        return SearchResult(D, I)

    def search_device(self, qbuf: N.DeviceBuffer, nq: int, k: int, Dbuf: N.DeviceBuffer,
                      Ibuf: N.DeviceBuffer, dtype: int = N.VS_DTYPE_F32) -> None:
        """Queries and results resident in device memory."""
        N.check(self._lib.vs_index_search_device(self._h, qbuf.ptr, dtype, int(nq), int(k), Dbuf.ptr,
                                                 Ibuf.ptr))

    def search_subsets(self, queries, k: int, ids, seg_off, seg_len) -> SearchResult:
        """Exact top-k of each query over its own row subsets: query i scans
        ids[seg_off[i, s] : seg_off[i, s] + seg_len[i, s]] for every s (the
        fine scan of IndexIVFFlat.search, index_ivf_flat.dart:131-170)."""
        q, code = _dtype_code(queries if isinstance(queries, np.ndarray) else as_rows(queries, self.d))
        nq = q.shape[0] if q.ndim == 2 else 0
        if nq == 0:
            return SearchResult(np.zeros((0, k), np.float32), np.zeros((0, k), np.int32))
        ids = np.ascontiguousarray(ids, np.int32)
        off = np.ascontiguousarray(seg_off, np.int64).reshape(nq, -1)
        ln = np.ascontiguousarray(seg_len, np.int64).reshape(nq, -1)
        D = np.empty((nq, k), np.float32)
        I = np.empty((nq, k), np.int32)
        vp = ctypes.c_void_p
        N.check(self._lib.vs_index_search_subsets(
            self._h, q.ctypes.data_as(vp), code, nq, int(k), ids.ctypes.data_as(vp), ids.size,
            off.ctypes.data_as(vp), ln.ctypes.data_as(vp), off.shape[1], D.ctypes.data_as(vp),
            I.ctypes.data_as(vp)))
        return SearchResult(D, I)

    def score_all(self, q) -> np.ndarray:
        """fp32 of the exact fp64 score of every stored row against q
        (l2sq / dot, index.dart:181-200)."""
        v = np.ascontiguousarray(q, np.float32).reshape(-1)
        if v.size != self.d:
            raise ValueError(f"query length {v.size} != {self.d}")
        out = np.empty(self.ntotal, np.float32)
        N.check(self._lib.vs_index_score_all(self._h, v.ctypes.data_as(ctypes.c_void_p),
                                             out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def range_search(self, queries, radius: float) -> RangeSearchResult:
        """index_flat.dart:99-137: dist <= radius (L2) or dot >= radius (IP), fp64 test."""
        q, code = _dtype_code(queries if isinstance(queries, np.ndarray) else as_rows(queries, self.d))
        nq = q.shape[0] if q.ndim == 2 else 0
        if nq and q.shape[1] != self.d:
            raise ValueError(f"query length {q.shape[1]} != {self.d}")
        out = ctypes.POINTER(N.RangeSearchC)()
        N.check(self._lib.vs_index_range_search(self._h, q.ctypes.data_as(ctypes.c_void_p), code, nq,
                                                float(radius), ctypes.byref(out)))
        try:
            r = out.contents
            lims = np.ctypeslib.as_array(r.lims, shape=(nq + 1,)).copy()
            tot = int(lims[-1])
            D = np.ctypeslib.as_array(r.D, shape=(max(tot, 1),))[:tot].copy()
            I = np.ctypeslib.as_array(r.I, shape=(max(tot, 1),))[:tot].copy()
        finally:
            self._lib.vs_range_result_free(out)
        return RangeSearchResult(lims, D, I)

    def self_join(self, threshold: float):
        """All pairs i < j whose score passes threshold, sorted by (i, j):
        the pair list of bin/vector_dedup_demo.dart:115-128."""
        out = ctypes.POINTER(N.PairsC)()
        N.check(self._lib.vs_index_self_join(self._h, float(threshold), ctypes.byref(out)))
        try:
            p = out.contents
            m = int(p.npairs)
            c = max(m, 1)
            i = np.ctypeslib.as_array(p.i, shape=(c,))[:m].copy()
            j = np.ctypeslib.as_array(p.j, shape=(c,))[:m].copy()
            s = np.ctypeslib.as_array(p.s, shape=(c,))[:m].copy()
        finally:
            self._lib.vs_pairs_free(out)
        return i, j, s

    # --- profiling (per-kernel HIP-event timing on the index's stream) ---
    def prof_enable(self, on: bool = True) -> None:
        N.check(self._lib.vs_prof_enable(self._h, 1 if on else 0))

    def prof_get(self, family: str) -> tuple[int, float]:
        n = ctypes.c_int64(0)
        ms = ctypes.c_double(0.0)
        N.check(self._lib.vs_prof_get(self._h, family.encode(), ctypes.byref(n), ctypes.byref(ms)))
        return int(n.value), float(ms.value)

    def prof_reset(self) -> None:
        N.check(self._lib.vs_prof_reset(self._h))


def IndexFlatL2(d: int, **kw) -> GpuIndexFlat:
    """index_flat.dart:192, served by the GPU index."""
    return GpuIndexFlat.l2(d, **kw)


def IndexFlatIP(d: int, **kw) -> GpuIndexFlat:
    """index_flat.dart:196, served by the GPU index."""
    return GpuIndexFlat.ip(d, **kw)
