"""Lloyd k-means on the GPU flat path (lib/core/vector_store/kmeans.dart).

Each iteration is one library call (vs_kmeans_step) doing the reference's
assignment step (strict-'<' argmin over fp64 squared distances, fp64
objective in point order; kmeans.dart:91-105) and update step (fp32 running
sums in point order scaled by fp64 1/count, empty clusters copied from the
largest one plus jitter; kmeans.dart:107-140).

Initialisation is the reference's k-means++ (kmeans.dart:48-85): a uniform
first pick, closestSq = fp32 of the fp64 squared distance to the nearest
chosen centroid (refreshed on the GPU by vs_index_score_all after each
pick), the fp64 running sum in point order, target = u * sum and the first
point whose running sum reaches it, a uniform pick when the sum is 0.  The
one generator drives the picks and, in centroid order, the jitter of empty
clusters only (each step's unused draws are rewound).  The generator is
numpy's Philox: dart:math Random's stream cannot be reproduced outside the
Dart VM, so the picks differ from the reference's; the arithmetic does not.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _native as N
from .gpu_index_flat import GpuIndexFlat
from .index import Metric


@dataclass
class KmeansResult:
    """kmeans.dart:12-23."""

    centroids: np.ndarray  # (k, d) float32
    assignments: np.ndarray  # (n,) int32
    objective: float


def kmeans_step(points: GpuIndexFlat, centroids: np.ndarray, min_points: int = 1,
                jitter_u: np.ndarray | None = None, out=None):
    """One Lloyd iteration.  Returns (assign, new_centroids, counts, objective).

    out: optional (assign int32 [n], centroids float32 [K, d], counts int32
    [K]) C-contiguous arrays the results are written to (as the reference's
    train loop reuses its assignment buffer across iterations)."""
    cen = np.ascontiguousarray(centroids, dtype=np.float32)
    K, d = cen.shape
    n = points.ntotal
    if out is None:
        assign = np.empty(n, np.int32)
        out_c = np.empty((K, d), np.float32)
        counts = np.empty(K, np.int32)
    else:
        assign, out_c, counts = out
        for arr, dt, shape in ((assign, np.int32, (n,)), (out_c, np.float32, (K, d)),
                               (counts, np.int32, (K,))):
            if arr.dtype != dt or arr.shape != shape or not arr.flags.c_contiguous:
                raise ValueError(f"out array {arr.dtype} {arr.shape}: need C-contiguous {dt} {shape}")
    out = out_c
    obj = ctypes.c_double(0.0)
    ju = np.ascontiguousarray(jitter_u if jitter_u is not None else np.zeros(0), dtype=np.float64)
    N.check(points._lib.vs_kmeans_step(points.handle, cen.ctypes.data_as(ctypes.c_void_p), K,
                                       int(min_points), ju.ctypes.data_as(ctypes.c_void_p), ju.size,
                                       assign.ctypes.data_as(ctypes.c_void_p),
                                       out.ctypes.data_as(ctypes.c_void_p),
                                       counts.ctypes.data_as(ctypes.c_void_p), ctypes.byref(obj)))
    return assign, out, counts, float(obj.value)


def kmeans_pp_init(points: GpuIndexFlat, x: np.ndarray, k: int, rng) -> np.ndarray:
    """k-means++ seeding (kmeans.dart:48-85) with the points resident in
    `points` (fp32 storage, the rows of x); rng.integers / rng.random stand
    for Random.nextInt / nextDouble."""
    n, d = x.shape
    cen = np.empty((k, d), np.float32)
    cen[0] = x[int(rng.integers(n))]
    closest = points.score_all(cen[0])  # Float32List closestSq (fp32 of the fp64 sum)
    for c in range(1, k):
        acc = np.cumsum(closest, dtype=np.float64)  # sum += closestSq[i], in point order
        total = float(acc[-1])
        if total <= 0:
            cen[c] = x[int(rng.integers(n))]
        else:
            target = rng.random() * total
            pick = int(np.searchsorted(acc, target, side="left"))  # first acc >= target
            cen[c] = x[min(pick, n - 1)]
        # dsq < closestSq[i] on the fp64 value stores fp32(dsq): the fp32 minimum
        closest = np.minimum(closest, points.score_all(cen[c]))
    return cen


class Kmeans:
    """kmeans.dart:26-41: Kmeans(d, k, niter=20, seed=1234, minPointsPerCentroid=1)."""

    def __init__(self, d: int, k: int, niter: int = 20, seed: int = 1234,
                 min_points_per_centroid: int = 1, verbose: bool = False, device: int = 0):
        self.d, self.k, self.niter, self.seed = int(d), int(k), int(niter), int(seed)
        self.min_points_per_centroid = int(min_points_per_centroid)
        self.verbose = verbose
        self.device = device

    def train(self, xs, init_centroids: np.ndarray | None = None) -> KmeansResult:
        x = np.ascontiguousarray(xs, dtype=np.float32)
        n = x.shape[0]
        if n < self.k:
            raise ValueError(f"k-means: need at least k={self.k} vectors, got {n}")
        rng = np.random.Generator(np.random.Philox(self.seed))
        pts = GpuIndexFlat(self.d, Metric.l2, storage="f32", device=self.device)
        try:
            pts.add(x)
            if init_centroids is None:
                cen = kmeans_pp_init(pts, x, self.k, rng)
            else:
                cen = np.ascontiguousarray(init_centroids, dtype=np.float32).copy()
            assign = np.zeros(n, np.int32)
            obj = 0.0
            for it in range(self.niter):
                # the step takes jitter draws for its empty clusters, in
                # centroid order: offer k * d of them, then advance the
                # generator by only as many as were used
                state = rng.bit_generator.state
                offer = rng.random(self.k * self.d)
                assign, cen, counts, obj = kmeans_step(pts, cen, self.min_points_per_centroid, offer)
                used = int(np.count_nonzero(counts < self.min_points_per_centroid)) * self.d
                rng.bit_generator.state = state
                rng.random(used)
                if self.verbose:
                    print(f"  k-means iter {it} obj={obj:.4f}")
        finally:
            pts.close()
        return KmeansResult(cen, assign, obj)
