"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is chosen so a plausible mistake fails it:
  - numpy fp64 brute force (BLAS summation order) on small random inputs;
  - closed forms (orthonormal basis, integer grids with exact distances);
  - the reference fixtures (data/*/index.bin) against numpy-derived goldens;
  - hand-derived cases of the reference's quirks: the fp32-stored heap root
    with strict acceptance (index.dart:248-260), the fp64 range test before
    fp32 storage (index_flat.dart:115-132), unfused fp64 multiply-add in the
    L2 sum (index_flat.dart:80-83), lowest-index argmin (kmeans.dart:96-101),
    sequential fp32 cluster sums (kmeans.dart:110-118).
"""
import json
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle
from vector_store import synthetic as syn

HERE = os.path.dirname(os.path.abspath(__file__))


def np_scores(xb, xq, metric):
    b = xb.astype(np.float64)
    q = xq.astype(np.float64)
    if metric == oracle.L2:
        return ((q[:, None, :] - b[None, :, :]) ** 2).sum(-1)
    return q @ b.T


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
@pytest.mark.parametrize("nthreads", [1, 3])
def test_brute_force_numpy(metric, nthreads):
    g = syn.rng(11, metric)
    xb = g.standard_normal((700, 13)).astype(np.float32)
    xq = g.standard_normal((9, 13)).astype(np.float32)
    D, I = oracle.flat_search(xb, xq, 7, metric, nthreads)
    s = np_scores(xb, xq, metric)
    order = np.argsort(s if metric == oracle.L2 else -s, axis=1, kind="stable")[:, :7]
    assert np.array_equal(I, order)
    ref = np.take_along_axis(s, order, 1)
    # two fp64 summation orders differ far below fp32 resolution
    assert np.allclose(D, ref.astype(np.float32), rtol=2e-7, atol=1e-7)


def test_orthonormal_closed_form():
    e = np.eye(16, dtype=np.float32)
    D, I = oracle.flat_search(e, e, 2, oracle.IP)
    assert np.array_equal(I[:, 0], np.arange(16)) and np.all(D[:, 0] == 1.0) and np.all(D[:, 1] == 0.0)
    D, I = oracle.flat_search(e, e, 2, oracle.L2)
    assert np.all(D[:, 0] == 0.0) and np.all(D[:, 1] == 2.0)
    # Ties at distance 2 follow the heap (index.dart:248-299), traced by hand
    # for k = 2: query 0 keeps [0, 1]; query 1 pushes (2, id0), (0, id1) and
    # then rejects the equal scores; query i >= 2 holds [(2, id0), (2, id1)]
    # until (0, id i) replaces the root id 0, leaving id 1.
    assert np.array_equal(I[:, 1], np.where(np.arange(16) == 1, 0, 1))


def test_integer_grid_exact():
    xb = syn.int_grid(2000, 128, 5, 0)
    xq = syn.int_grid(4, 128, 5, 1)
    D, I = oracle.flat_search(xb, xq, 50, oracle.L2)
    exact = ((xq[:, None, :].astype(np.int64) - xb[None].astype(np.int64)) ** 2).sum(-1)
    for q in range(4):
        assert np.array_equal(D[q], np.sort(exact[q])[:50].astype(np.float32))
        assert np.all(exact[q][I[q]] == D[q])


def test_sentinels_and_ties():
    xb = np.ones((3, 4), np.float32)
    D, I = oracle.flat_search(xb, xb[:1], 5, oracle.L2)
    assert list(I[0]) == [0, 1, 2, -1, -1] and np.all(D[0, 3:] == np.inf)
    D, I = oracle.flat_search(xb, xb[:1], 5, oracle.IP)
    assert np.all(D[0, 3:] == -np.inf)
    # k = 0 with a non-empty index throws in the reference
    with pytest.raises(ValueError):
        oracle.flat_search(xb, xb[:1], 0, oracle.L2)


def test_heap_root_is_fp32_strict():
    """Rows x0 = (1 + 2^-23, 0), x1 = (1, 2^-11), query 0: fp64 scores are
    A = 1 + 2^-22 + 2^-46 and B = 1 + 2^-22 < A.  The heap stores fp32(A) =
    1 + 2^-22 = B, so B is not strictly better and x1 is rejected: the
    reference answers id 0 where an fp64-exact heap would answer id 1."""
    xb = np.array([[1 + 2.0 ** -23, 0], [1, 2.0 ** -11]], np.float32)
    D, I = oracle.flat_search(xb, np.zeros((1, 2), np.float32), 1, oracle.L2)
    assert I[0, 0] == 0 and D[0, 0] == np.float32(1 + 2.0 ** -22)


def test_range_compares_fp64_before_rounding():
    """q = x = (1 + 2^-23): s = A = 1 + 2^-22 + 2^-46 in fp64 while fp32(A) =
    1 + 2^-22 < A.  radius = A keeps the hit (fp64 test, inclusive); a test on
    the stored fp32 value would drop it.  radius just above A drops it."""
    v = np.array([[1 + 2.0 ** -23]], np.float32)
    A = (1 + 2.0 ** -23) ** 2
    lims, D, I = oracle.flat_range_search(v, v, A, oracle.IP)
    assert list(lims) == [0, 1] and D[0] == np.float32(1 + 2.0 ** -22)
    lims, D, I = oracle.flat_range_search(v, v, np.nextafter(A, 2.0), oracle.IP)
    assert list(lims) == [0, 0]
    # L2 is inclusive too: distance 0 within radius 0
    lims, _, _ = oracle.flat_range_search(v, v, 0.0, oracle.L2)
    assert list(lims) == [0, 1]


def test_range_equals_filtered_knn():
    """vector_store_test.dart:307-329 restated."""
    g = syn.rng(3, 3)
    xb = g.standard_normal((400, 16)).astype(np.float32)
    xq = g.standard_normal((20, 16)).astype(np.float32)
    D, I = oracle.flat_search(xb, xq, 400, oracle.L2)
    radius = float((np.float64(D[0, 2]) + np.float64(D[0, 3])) / 2)
    lims, RD, RI = oracle.flat_range_search(xb, xq, radius, oracle.L2, 4)
    s = np_scores(xb, xq, oracle.L2)
    for q in range(20):
        exp = np.nonzero(s[q] <= radius)[0]
        assert np.array_equal(RI[lims[q]:lims[q + 1]], exp)  # ascending id order


def _py_l2(a, b):
    """The reference's loop in Python floats (IEEE doubles, no contraction)."""
    s = 0.0
    for x, y in zip(a.tolist(), b.tolist()):
        diff = x - y
        s += diff * diff
    return s


def _py_l2_fused(a, b):
    s = Fraction(0)
    out = 0.0
    for x, y in zip(a.tolist(), b.tolist()):
        diff = x - y
        out = float(Fraction(out) + Fraction(diff) * Fraction(diff))  # one rounding
    return out


def test_l2_sum_is_unfused_fp64():
    """kmeans_assign reports each point's fp64 squared distance: it must equal
    the reference's separate multiply and add, and the case is chosen so a
    fused multiply-add gives a different fp64 value."""
    g = syn.rng(5, 5)
    for trial in range(200):
        x = (g.standard_normal((1, 40)) * 2.0 ** g.integers(-30, 5, size=40)).astype(np.float32)
        c = g.standard_normal((1, 40)).astype(np.float32)
        if _py_l2(x[0], c[0]) != _py_l2_fused(x[0], c[0]):
            break
    else:
        pytest.skip("no discriminating case found")
    _, best, obj = oracle.kmeans_assign(x, c)
    assert best[0] == _py_l2(x[0], c[0]) != _py_l2_fused(x[0], c[0])


def test_kmeans_assign_lowest_index_and_brute_force():
    g = syn.rng(8, 1)
    x = g.standard_normal((500, 12)).astype(np.float32)
    cen = np.concatenate([x[:10], x[:10]]).astype(np.float32)  # exact duplicate centroids
    a, best, obj = oracle.kmeans_assign(x, cen, 2)
    s = np_scores(cen, x, oracle.L2)
    assert np.array_equal(a, np.argmin(s, axis=1))  # argmin returns the first (lowest) index
    assert np.all(a < 10)
    assert obj == sum(best.tolist())  # fp64 sum in point order


def test_kmeans_update_sequential_fp32():
    """Cluster 0 gets points [1, 2^-24, 2^-24, 2^-24] in that order: each fp32
    add of 2^-24 to 1 rounds back to 1 (tie to even), so the sum is 1 and the
    mean 0.25; pairwise summation would give 1 + 3 * 2^-24."""
    x = np.array([[1.0], [2.0 ** -24], [2.0 ** -24], [2.0 ** -24], [5.0]], np.float32)
    assign = np.array([0, 0, 0, 0, 1], np.int32)
    cen, counts, used = oracle.kmeans_update(x, assign, np.zeros((2, 1), np.float32))
    assert list(counts) == [4, 1] and used == 0
    assert cen[0, 0] == np.float32(0.25) and cen[1, 0] == 5.0
    # mean uses fp64 1/count then one rounding: 1/3 of 1.0
    x3 = np.array([[1.0], [0.0], [0.0]], np.float32)
    cen, _, _ = oracle.kmeans_update(x3, np.zeros(3, np.int32), np.zeros((1, 1), np.float32))
    assert cen[0, 0] == np.float32(1.0 * (1.0 / 3.0))


def test_kmeans_update_empty_cluster_in_place():
    """kmeans.dart:127-139: an empty cluster copies the largest cluster's
    centroid as it is at that moment (already updated when it precedes) plus
    (u - 0.5) * 1e-4."""
    x = np.array([[0.0], [2.0], [4.0], [10.0]], np.float32)
    assign = np.array([1, 1, 1, 2], np.int32)  # cluster 0 empty, 1 is the largest
    cen_in = np.array([[100.0], [7.0], [8.0], [50.0]], np.float32)  # cluster 3 empty too
    u = np.array([0.75, 0.25])
    cen, counts, used = oracle.kmeans_update(x, assign, cen_in, 1, u)
    assert used == 2 and list(counts) == [0, 3, 1, 0]
    # c = 0 runs before cluster 1 is updated: copies the OLD centroid 7.0
    assert cen[0, 0] == np.float32(7.0 + 0.25 * 1e-4)
    assert cen[1, 0] == np.float32(2.0)
    # c = 3 runs after: copies the NEW centroid 2.0
    assert cen[3, 0] == np.float32(2.0 - 0.25 * 1e-4)


def test_self_join_matches_range_filter():
    x = syn.dedup_set(600, 32, 0.1, 0.05, 9)
    i, j, s = oracle.self_join(x, 0.9, nthreads=3)
    lims, D, I = oracle.flat_range_search(x, x, 0.9, oracle.IP, 2)
    pairs = [(q, int(t)) for q in range(len(x)) for t in I[lims[q]:lims[q + 1]] if t > q]
    assert list(zip(i.tolist(), j.tolist())) == pairs
    assert len(pairs) > 10


def test_reference_fixtures_against_numpy_goldens():
    from vector_store import io as vio

    gold = json.load(open(os.path.join(HERE, "golden", "flat_fixtures.json")))
    for name, g in gold.items():
        hdr, x = vio.read_faisdart_flat(os.path.join(HERE, "golden", name))
        assert hdr["metric"] == g["metric"] == 1
        D, I = oracle.flat_search(x, x, 5, oracle.IP, 2)
        assert np.array_equal(I, np.array(g["top5_ids"]))
        assert np.allclose(D, np.array(g["top5_scores_f64"], np.float32), rtol=2e-7, atol=1e-7)
        assert np.array_equal(I[:, 0], np.arange(hdr["ntotal"]))  # self top-1
        # thresholds between observed similarities give exact pair sets
        m = g["max_offdiag"]
        lims, _, _ = oracle.flat_range_search(x, x, m + 1e-6, oracle.IP)
        assert np.array_equal(np.diff(lims), np.ones(hdr["ntotal"]))


@pytest.mark.parametrize("metric", [oracle.L2, oracle.IP])
def test_range_search_brute_force_numpy(metric):
    """Range search at d > 1 with n not a multiple of 4 (the oracle's scalar
    tail): hits = numpy fp64 scores against the radius, ids ascending."""
    g = syn.rng(13, metric)
    xb = g.standard_normal((701, 37)).astype(np.float32)
    xq = g.standard_normal((11, 37)).astype(np.float32)
    s = np_scores(xb, xq, metric)
    radius = float(np.quantile(s, 0.02 if metric == oracle.L2 else 0.98))
    lims, D, I = oracle.flat_range_search(xb, xq, radius, metric, 3)
    for q in range(len(xq)):
        want = np.nonzero(s[q] <= radius if metric == oracle.L2 else s[q] >= radius)[0]
        got = I[lims[q]:lims[q + 1]]
        assert np.array_equal(got, want)
        assert np.allclose(D[lims[q]:lims[q + 1]], s[q][want].astype(np.float32), rtol=2e-7,
                           atol=1e-6)


def test_self_join_brute_force_numpy():
    """IP self-join at d = 29, n = 513: every pair i < j with fp64 dot >= t,
    sorted by (i, j), against numpy (vector_dedup_demo.dart:115-128)."""
    x = syn.dedup_set(513, 29, 0.1, 0.05, 4)
    s = x.astype(np.float64) @ x.astype(np.float64).T
    t = 0.8
    ii, jj = np.nonzero(np.triu(s >= t, k=1))
    i, j, sc = oracle.self_join(x, t, nthreads=2)
    assert np.array_equal(i, ii) and np.array_equal(j, jj) and len(i) > 20
    assert np.allclose(sc, s[ii, jj].astype(np.float32), rtol=2e-7)


def test_oracle_memory_safety_under_sanitizers():
    """oracle.c under AddressSanitizer + UndefinedBehaviorSanitizer: a driver
    (oracle/asan_check.c) calls every entry point on edge shapes (ragged d,
    counts not multiples of 4, k above n, empty inputs, growing range
    buffers, self-join windows, empty k-means clusters); any invalid access
    aborts the run with the sanitizer's report."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("no gcc to build the sanitizer run")
    odir = os.path.join(os.path.dirname(HERE), "oracle")
    b = subprocess.run(["make", "-s", "-C", odir, "asan"], capture_output=True, text=True)
    if b.returncode != 0 and "asan" in (b.stderr + b.stdout).lower() and "cannot find" in b.stderr:
        pytest.skip("this gcc has no sanitizer runtime")
    assert b.returncode == 0, b.stderr
    r = subprocess.run([os.path.join(odir, "asan_check")], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "asan_check ok" in r.stdout
