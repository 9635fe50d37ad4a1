"""k-means step parity (kmeans.dart:91-140) against the oracle with identical
input centroids: assignments equal (strict '<', lowest index on ties),
objective and updated centroids bit-identical (same fp64 scores, same fp32
running sums in point order)."""
import numpy as np
import pytest

import oracle
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def test_kmeans_step_parity(vs):
    x, _ = syn.gaussian_mixture(20_000, 256, 64, 0.1, 1234)
    cen = x[syn.seeded_subset(len(x), 256, 1234)].copy()
    pts = vs.GpuIndexFlat.l2(256, storage="f32")
    pts.add(x)
    for it in range(3):
        u = syn.rng(77, it).random(256 * 256)  # jitter draws (an empty cluster appears at it = 1)
        a, newc, cnt, obj = vs.kmeans_step(pts, cen, 1, u)
        ar, br, objr = oracle.kmeans_assign(x, cen, NT)
        assert np.array_equal(a, ar), f"iteration {it}: {np.sum(a != ar)} assignments differ"
        assert obj == objr
        cr, cntr, _ = oracle.kmeans_update(x, ar, cen, 1, u)
        assert np.array_equal(cnt, cntr)
        assert np.array_equal(newc.view(np.uint32), cr.view(np.uint32))
        cen = newc


def test_kmeans_empty_cluster_jitter(vs):
    """Centroids far from every point get no points: they copy the largest
    cluster plus (u - 0.5) * 1e-4 with u taken in order (kmeans.dart:127-139)."""
    x, _ = syn.gaussian_mixture(3000, 32, 4, 0.1, 7)
    cen = np.concatenate([x[:6], np.full((2, 32), 1e3, np.float32)]).astype(np.float32)
    u = syn.rng(1, 0).random(2 * 32)
    pts = vs.GpuIndexFlat.l2(32, storage="f32")
    pts.add(x)
    a, newc, cnt, obj = vs.kmeans_step(pts, cen, 1, u)
    ar, _, objr = oracle.kmeans_assign(x, cen, NT)
    cr, cntr, used = oracle.kmeans_update(x, ar, cen, 1, u)
    assert used == 64 and np.array_equal(a, ar) and obj == objr
    assert np.array_equal(newc.view(np.uint32), cr.view(np.uint32))


def test_kmeans_empty_cluster_before_largest(vs):
    """An empty cluster preceding the largest one copies the largest
    cluster's old centroid (the in-place loop of kmeans.dart:107-140 has not
    updated it yet); one after it copies the new centroid.  The oracle
    updates in place the same way; the centroids must be bit-identical."""
    g = syn.rng(9, 0)
    a_pts = (g.standard_normal((500, 16)) * 0.1).astype(np.float32)
    b_pts = (g.standard_normal((2000, 16)) * 0.1 + 5.0).astype(np.float32)
    x = np.concatenate([a_pts, b_pts]).astype(np.float32)
    far = np.full((1, 16), 1e3, np.float32)
    cen = np.concatenate([far, x[:1] + 0.3, x[600:601] + 0.3, far * 2]).astype(np.float32)
    u = syn.rng(9, 1).random(2 * 16)
    pts = vs.GpuIndexFlat.l2(16, storage="f32")
    pts.add(x)
    a, newc, cnt, obj = vs.kmeans_step(pts, cen, 1, u)
    ar, _, objr = oracle.kmeans_assign(x, cen, NT)
    cr, cntr, used = oracle.kmeans_update(x, ar, cen, 1, u)
    assert list(cntr) == [0, 500, 2000, 0] and used == 32
    assert np.array_equal(a, ar) and obj == objr and np.array_equal(cnt, cntr)
    assert np.array_equal(newc.view(np.uint32), cr.view(np.uint32))
    # the first empty cluster took the largest cluster's old centroid
    assert np.abs(newc[0] - cen[2]).max() < 1e-3 and np.abs(newc[3] - cr[2]).max() < 1e-3


def _rejitter(cen_old, newc, counts, min_points, u):
    """The Dart drop-in's GpuKmeans update of empty clusters: after a step
    with neutral jitter (u = 0.5, a plain copy), each cluster below
    min_points, in centroid order, becomes the largest cluster's centroid
    (its new value when it precedes, its old one otherwise) plus
    (u - 0.5) * 1e-4 in fp64, rounded to fp32 -- the draws taken in order."""
    out = newc.copy()
    big = int(np.argmax(counts))  # the first of the largest count
    t = 0
    for c in range(len(counts)):
        if counts[c] >= min_points:
            continue
        src = out[big] if big < c else cen_old[big]
        for j in range(out.shape[1]):
            out[c, j] = np.float32(np.float64(src[j]) + (u[t] - 0.5) * 1e-4)
            t += 1
    return out


@pytest.mark.parametrize("min_points", [1, 600])
def test_kmeans_neutral_jitter_then_host_jitter(vs, min_points):
    """The GpuKmeans of the Dart drop-in draws the jitter from dart:math
    Random itself: it runs each step with neutral jitter and re-jitters the
    clusters below minPointsPerCentroid on the host.  That equals a step
    given the same draws directly, bit for bit, with empty clusters before
    and after the largest one (min_points 600 also replaces a small
    non-empty cluster)."""
    g = syn.rng(9, 0)
    a_pts = (g.standard_normal((500, 16)) * 0.1).astype(np.float32)
    b_pts = (g.standard_normal((2000, 16)) * 0.1 + 5.0).astype(np.float32)
    x = np.concatenate([a_pts, b_pts]).astype(np.float32)
    far = np.full((1, 16), 1e3, np.float32)
    cen = np.concatenate([far, x[:1] + 0.3, x[600:601] + 0.3, far * 2]).astype(np.float32)
    u = syn.rng(9, 2).random(4 * 16)
    pts = vs.GpuIndexFlat.l2(16, storage="f32")
    pts.add(x)
    a1, direct, cnt1, obj1 = vs.kmeans_step(pts, cen, min_points, u)
    a2, neutral, cnt2, obj2 = vs.kmeans_step(pts, cen, min_points, np.full(4 * 16, 0.5))
    pts.close()
    assert np.array_equal(a1, a2) and obj1 == obj2 and np.array_equal(cnt1, cnt2)
    host = _rejitter(cen, neutral, cnt2, min_points, u)
    assert np.array_equal(host.view(np.uint32), direct.view(np.uint32))
    _, _, used = oracle.kmeans_update(x, a1, cen, min_points, u)
    assert used == 16 * int(np.sum(cnt1 < min_points)) and used >= 32


def test_kmeans_train_monotone(vs):
    """vector_store_test.dart:91-111: re-assignment objective <= 1.05 x training objective."""
    x, _ = syn.gaussian_mixture(400, 16, 8, 0.05, 1)
    res = vs.Kmeans(16, 8, niter=30).train(x)
    assert res.centroids.shape == (8, 16) and res.assignments.shape == (400,)
    _, _, reobj = oracle.kmeans_assign(x, res.centroids, 1)
    assert reobj <= res.objective * 1.05 + 1e-6


def test_kmeans_prepared_points_follow_adds(vs):
    """The points prepared for the assign scan are kept across iterations;
    adding rows (or removing some) must invalidate them: each step still
    equals the oracle on the index's current rows."""
    x, _ = syn.gaussian_mixture(5000, 64, 8, 0.1, 3)
    cen = x[:16].copy()
    pts = vs.GpuIndexFlat.l2(64, storage="f32")
    pts.add(x[:3000])
    a1, _, _, o1 = vs.kmeans_step(pts, cen, 1, syn.rng(4, 0).random(16 * 64))
    ar1, _, or1 = oracle.kmeans_assign(x[:3000], cen, NT)
    assert np.array_equal(a1, ar1) and o1 == or1
    pts.add(x[3000:])
    a2, _, _, o2 = vs.kmeans_step(pts, cen, 1, syn.rng(4, 1).random(16 * 64))
    ar2, _, or2 = oracle.kmeans_assign(x, cen, NT)
    assert np.array_equal(a2, ar2) and o2 == or2
    pts.remove_ids(list(range(0, 5000, 2)))
    a3, _, _, o3 = vs.kmeans_step(pts, cen, 1, syn.rng(4, 2).random(16 * 64))
    ar3, _, or3 = oracle.kmeans_assign(x[1::2], cen, NT)
    assert np.array_equal(a3, ar3) and o3 == or3
    pts.close()


def test_kmeans_step_in_place_buffers(vs):
    """vs_kmeans_step with centroids_out the same buffer as centroids_in (the
    in-place update of kmeans.dart:107-140): the same centroids as with
    separate buffers, empty clusters included (their old centroids are read
    after the new ones are written)."""
    import ctypes
    from vector_store import _native as N

    g = syn.rng(9, 0)
    a_pts = (g.standard_normal((500, 16)) * 0.1).astype(np.float32)
    b_pts = (g.standard_normal((2000, 16)) * 0.1 + 5.0).astype(np.float32)
    x = np.concatenate([a_pts, b_pts]).astype(np.float32)
    far = np.full((1, 16), 1e3, np.float32)
    cen = np.concatenate([far, x[:1] + 0.3, x[600:601] + 0.3, far * 2]).astype(np.float32)
    u = syn.rng(9, 1).random(2 * 16)
    pts = vs.GpuIndexFlat.l2(16, storage="f32")
    pts.add(x)
    _, sep, cnt_sep, obj_sep = vs.kmeans_step(pts, cen, 1, u)
    inout = cen.copy()
    assign = np.empty(len(x), np.int32)
    cnt = np.empty(4, np.int32)
    obj = ctypes.c_double(0.0)
    p = inout.ctypes.data_as(ctypes.c_void_p)
    N.check(pts._lib.vs_kmeans_step(pts.handle, p, 4, 1, u.ctypes.data_as(ctypes.c_void_p), u.size,
                                    assign.ctypes.data_as(ctypes.c_void_p), p,
                                    cnt.ctypes.data_as(ctypes.c_void_p), ctypes.byref(obj)))
    pts.close()
    assert np.array_equal(cnt, cnt_sep) and obj.value == obj_sep and np.sum(cnt == 0) == 2
    assert np.array_equal(inout.view(np.uint32), sep.view(np.uint32))


@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_kmeans_nonfinite_centroids(vs, bad):
    """Centroids holding NaN or infinity: the step reports VS_ERR_NONFINITE
    (checked with the pick's results, before any exhaustive pass), and the
    next step on the same points with finite centroids equals the oracle's."""
    from vector_store import _native as N

    x, _ = syn.gaussian_mixture(20_000, 256, 64, 0.1, 91)
    cen = x[syn.seeded_subset(len(x), 256, 91)].copy()
    pts = vs.GpuIndexFlat.l2(256, storage="f32")
    pts.add(x)
    u = syn.rng(92, 0).random(256 * 256)
    a, c1, _, _ = vs.kmeans_step(pts, cen, 1, u)  # a previous step (running minima, order)
    badc = c1.copy()
    badc[17, 5] = bad
    with pytest.raises(N.VsError) as ei:
        vs.kmeans_step(pts, badc, 1, u)
    assert ei.value.code == N.VS_ERR_NONFINITE
    a2, c2, cnt2, obj2 = vs.kmeans_step(pts, c1, 1, u)
    pts.close()
    ar, _, objr = oracle.kmeans_assign(x, c1, NT)
    cr, cntr, _ = oracle.kmeans_update(x, ar, c1, 1, u)
    assert np.array_equal(a2, ar) and obj2 == objr and np.array_equal(cnt2, cntr)
    assert np.array_equal(c2.view(np.uint32), cr.view(np.uint32))
