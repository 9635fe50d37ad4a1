"""Parity of the row-shared scan (large query batches over bf16 rows of 128
or 256 elements; each workgroup stages its row tiles in LDS once for four
waves of register-resident queries) against the CPU oracle (restating
IndexFlat.search, index_flat.dart:62-97).

Row counts end inside a row tile and inside a split, query counts inside a
query block, d is ragged below the stored row length, both metrics, k from
1 to 400 and k above the row count.  Each test checks, through the always-on
"shared" launch counter, that the row-shared kernel really ran."""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


@pytest.fixture(autouse=True)
def _share(opts):
    """The row-shared scan is on for both row lengths in every test here."""
    opts(share=1)


def _search(vs, xb, xq, k, metric, storage="auto", expect_shared=True):
    idx = vs.GpuIndexFlat(xb.shape[1], vs.Metric(metric), storage=storage)
    idx.add(xb)
    r = idx.search(xq, k)
    n, _ = idx.prof_get("shared")
    idx.close()
    if expect_shared:
        assert n >= 1, "the row-shared scan did not run"
    return r.distances, r.ids


@pytest.mark.parametrize("n,d,nq,k,metric", [
    (5000, 128, 300, 10, 0),
    (4097, 100, 257, 100, 1),
    (300, 16, 512, 1, 0),
    (50, 64, 256, 100, 0),        # k > n: sentinels
    (20011, 128, 1000, 400, 1),  # kk_final 512
    (3001, 200, 300, 10, 0),     # rows of 256 elements
    (9000, 256, 600, 100, 1),
])
def test_integer_rows_exact(vs, n, d, nq, k, metric):
    """Integer rows 0..255 are bf16-exact, so every accumulator is an exact
    integer: the result is bit-identical to the oracle's (ties aside)."""
    xb = syn.int_grid(n, d, 3, 0)
    xq = syn.int_grid(nq, d, 3, 1)
    D, I = _search(vs, xb, xq, k, metric)
    Dr, Ir = oracle.flat_search(xb, xq, k, metric, NT)
    assert_knn_parity(D, I, Dr, Ir, metric, rtol=0.0, atol=0.0, xb=xb, xq=xq)


@pytest.mark.parametrize("metric", [0, 1])
def test_bf16_unit_vectors(vs, metric):
    """bf16 storage of unit vectors with bf16 queries (one query plane); the
    oracle sees the stored bf16 values upcast to fp32."""
    xb16 = syn.to_bf16_bits(syn.normal_unit(30_000, 128, 21, 0))
    xq16 = syn.to_bf16_bits(syn.normal_unit(700, 128, 21, 1))
    D, I = _search(vs, xb16, xq16, 10, metric, storage="bf16")
    Dr, Ir = oracle.flat_search(syn.bf16_bits_to_f32(xb16), syn.bf16_bits_to_f32(xq16), 10,
                                metric, NT)
    assert_knn_parity(D, I, Dr, Ir, metric, rtol=1e-5)


def test_matches_streaming_scan_large(vs, opts):
    """configs[1] shape on a 300k-row slice (estimated thresholds active):
    the row-shared scan returns the same distances as the streaming scan,
    and the oracle's on a query sample."""
    xb = syn.int_grid(300_000, 128, 4, 0)
    xq = syn.int_grid(1024, 128, 4, 1)
    D1, I1 = _search(vs, xb, xq, 100, 0)
    opts(share=0)
    D0, I0 = _search(vs, xb, xq, 100, 0, expect_shared=False)
    assert np.array_equal(D1, D0)
    sub = np.arange(0, 1024, 31)
    Dr, Ir = oracle.flat_search(xb, xq[sub], 100, 0, NT)
    assert_knn_parity(D1[sub], I1[sub], Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq[sub])


def test_small_batch_not_shared(vs):
    """Below the batch threshold the streaming scan runs instead."""
    xb = syn.int_grid(2000, 128, 5, 0)
    xq = syn.int_grid(100, 128, 5, 1)
    D, I = _search(vs, xb, xq, 10, 0, expect_shared=False)
    Dr, Ir = oracle.flat_search(xb, xq, 10, 0, NT)
    assert_knn_parity(D, I, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)


def _kmeans_check(vs, x, cen, min_points=1, seed=0, expect_fallback=False):
    pts = vs.GpuIndexFlat.l2(x.shape[1], storage="f32")
    pts.add(x)
    K = len(cen)
    u = syn.rng(seed + 1, 0).random(K * x.shape[1])
    a, newc, cnt, obj = vs.kmeans_step(pts, cen, min_points, u)
    shared, _ = pts.prof_get("shared")
    nfb, _ = pts.prof_get("kmeans_fallback_points")
    pts.close()
    assert shared >= 1, "the row-shared scan did not run"
    if expect_fallback:
        assert nfb >= 1
    ar, _, objr = oracle.kmeans_assign(x, cen, NT)
    assert np.array_equal(a, ar), f"{np.sum(a != ar)} assignments differ"
    assert obj == objr
    cr, cntr, _ = oracle.kmeans_update(x, ar, cen, min_points, u)
    assert np.array_equal(cnt, cntr)
    assert np.array_equal(newc.view(np.uint32), cr.view(np.uint32))
    return a


@pytest.mark.parametrize("n,d,ncomp,K", [(30_000, 256, 1024, 4096), (9_000, 100, 64, 500),
                                         (3_000, 256, 8, 20)])
def test_kmeans_register_shortlists(vs, n, d, ncomp, K):
    """k-means assign on the row-shared scan (fp32 points and centroids,
    one-pass bf16 selection): each scan lane appends the values below its
    running minimum + 2.5 bound to the point's list; the pick re-scores those
    within 2 bound of the smallest in fp64 and the rest are provably worse.
    Assignments, objective and centroids equal the oracle's (K = 20: lanes
    see few centroids each)."""
    x, _ = syn.gaussian_mixture(n, d, ncomp, 0.1, 41)
    cen = x[syn.seeded_subset(n, K, 41)].copy()
    _kmeans_check(vs, x, cen)


def test_kmeans_pick_beyond_distinct_bitmap(vs):
    """More than 16,384 centroids: the pick stages every lane's candidate
    slot by slot instead of numbering the wave's distinct candidates through
    its 16,384-bit map; the oracle's assignments, objective and centroids."""
    x, _ = syn.gaussian_mixture(18_000, 100, 64, 0.1, 47)
    cen = x[syn.seeded_subset(18_000, 17_000, 47)].copy()
    _kmeans_check(vs, x, cen)


def test_kmeans_register_shortlists_fallback(vs):
    """Forty copies of one centroid: more candidates within 2 bound of the
    smallest than the pick's 32 slots, so the exhaustive exact scan decides
    those points: the lowest index among the copies loses to the original
    (kmeans.dart:93-101)."""
    x, _ = syn.gaussian_mixture(6000, 256, 16, 0.1, 5)
    cen = x[syn.seeded_subset(len(x), 300, 5)].copy()
    cen[100:140] = cen[3]
    a = _kmeans_check(vs, x, cen, expect_fallback=True)
    assert not np.any((a >= 100) & (a < 140))


def test_kmeans_fallback_in_last_range_only(vs):
    """The pick runs over four consecutive point ranges and the objective's
    sequential sum starts on each range as soon as its pick ends; here only
    the last range's points have more tied candidates than the pick's 32
    slots, so the first three ranges are summed at once and the last after
    the exhaustive pass.  Assignments, objective (bit for bit) and centroids
    equal the oracle's, on that step and on the next one (grouped order)."""
    d = 256
    x1, _ = syn.gaussian_mixture(4500, d, 16, 0.1, 54)
    v = np.full(d, 3.0 / np.sqrt(d), np.float32) + x1.max()
    x2 = (v + 0.01 * syn.rng(55, 0).standard_normal((1500, d))).astype(np.float32)
    x = np.concatenate([x1, x2])
    cen = np.concatenate([x1[syn.seeded_subset(4500, 300, 54)], np.tile(v, (40, 1))])
    u = syn.rng(56, 0).random(len(cen) * d)
    idx = vs.GpuIndexFlat.l2(d, storage="f32")
    idx.add(x)
    c = cen
    for step in range(2):
        before = idx.prof_get("kmeans_fallback_points")[0]
        a, newc, cnt, obj = vs.kmeans_step(idx, c, 1, u)
        if step == 0:
            assert idx.prof_get("kmeans_fallback_points")[0] > before
        ar, cr, cntr, objr = _kmeans_oracle_step(x, c, u)
        assert np.array_equal(a, ar), f"step {step}: {np.sum(a != ar)} assignments differ"
        assert obj == objr and np.array_equal(cnt, cntr)
        assert np.array_equal(newc.view(np.uint32), cr.view(np.uint32))
        c = newc
    idx.close()


def test_kmeans_lists_full(vs):
    """Three hundred copies of one centroid overflow the points' k-means
    lists (more than cap - 16 appends): the lists are marked full and their
    points go to the exhaustive exact scan, whose argmin is the oracle's."""
    x, _ = syn.gaussian_mixture(4000, 256, 8, 0.1, 6)
    cen = x[syn.seeded_subset(len(x), 700, 6)].copy()
    cen[200:500] = cen[7]
    a = _kmeans_check(vs, x, cen, expect_fallback=True)
    assert not np.any((a >= 200) & (a < 500))


@pytest.mark.parametrize("km16,rt,nqb", [(0, 4, 2), (1, 2, 2), (1, 4, 4)])
def test_kmeans_lists_fp32_rows(vs, opts, km16, rt, nqb):
    """The k-means lists over the fp32 centroid rows rounded in the scan
    (option km16 = 0), or over their bf16 copy in 32-row tiles (km16_rt = 2)
    instead of 64-row ones, or with 64 points per wave (km16_nqb = 4, 32-row
    tiles; 30,000 points end inside a 256-point block): the oracle's
    assignments."""
    opts(km16=km16, km16_rt=rt, km16_nqb=nqb)
    x, _ = syn.gaussian_mixture(30_000, 256, 1024, 0.1, 44)
    cen = x[syn.seeded_subset(30_000, 4096, 44)].copy()
    _kmeans_check(vs, x, cen)


def _kmeans_oracle_step(x, cen, u):
    ar, _, objr = oracle.kmeans_assign(x, cen, NT)
    cr, cntr, _ = oracle.kmeans_update(x, ar, cen, 1, u)
    return ar, cr, cntr, objr


@pytest.mark.parametrize("nqb", [2, 4])
def test_kmeans_running_minima_from_last_step(vs, nqb):
    """Lloyd steps on one index: from the second step on, each point's
    running minimum in the assign scan starts at a bound from its previous
    centroid (previous squared distance, the centroid's shift, the
    accumulator bound), so its list holds what lies within the margin of
    the smallest accumulator.  Every step equals the oracle's step, and the
    same steps with the option kmin_init = 0."""
    x, _ = syn.gaussian_mixture(30_000, 256, 1024, 0.1, 48)
    cen = x[syn.seeded_subset(30_000, 4096, 48)].copy()
    u = syn.rng(49, 0).random(4096 * 256)
    a = vs.GpuIndexFlat.l2(256, storage="f32")
    b = vs.GpuIndexFlat.l2(256, storage="f32")
    a.add(x)
    b.add(x)
    b.set_option("kmin_init", 0)
    for g in (a, b):
        g.set_option("km16_nqb", nqb)
    a.prof_enable(True)
    c = cen
    for step in range(3):
        ra = vs.kmeans_step(a, c, 1, u)
        rb = vs.kmeans_step(b, c, 1, u)
        ar, cr, cntr, objr = _kmeans_oracle_step(x, c, u)
        assert np.array_equal(ra[0], ar), f"step {step}: {np.sum(ra[0] != ar)} assignments differ"
        assert ra[3] == objr and np.array_equal(ra[2], cntr)
        assert np.array_equal(ra[1].view(np.uint32), cr.view(np.uint32))
        assert np.array_equal(ra[0], rb[0]) and ra[3] == rb[3]
        c = ra[1]
    assert a.prof_get("kmin_init")[0] == 2
    assert b.prof_get("kmin_init")[0] == 0
    a.close()
    b.close()


def test_kmeans_running_minima_any_centroids(vs):
    """The starting bound holds for whatever centroids the next call brings
    (it only needs the previous centroid's shift): unrelated centroids,
    the same ones permuted, and after a change of K (no bound then, as
    after rows are added) all give the oracle's step."""
    x, _ = syn.gaussian_mixture(20_000, 256, 256, 0.1, 50)
    K = 1024
    u = syn.rng(51, 0).random(2 * K * 256)
    idx = vs.GpuIndexFlat.l2(256, storage="f32")
    idx.add(x)
    idx.prof_enable(True)
    steps = [x[syn.seeded_subset(20_000, K, 50)].copy(),
             x[syn.seeded_subset(20_000, K, 52)].copy()]  # unrelated
    steps.append(steps[1][::-1].copy())                     # permuted
    steps.append(x[syn.seeded_subset(20_000, K + 7, 53)].copy())  # K changes
    for i, c in enumerate(steps):
        r = vs.kmeans_step(idx, c, 1, u)
        ar, cr, cntr, objr = _kmeans_oracle_step(x, c, u)
        assert np.array_equal(r[0], ar), f"call {i}: {np.sum(r[0] != ar)} assignments differ"
        assert r[3] == objr and np.array_equal(r[1].view(np.uint32), cr.view(np.uint32))
    assert idx.prof_get("kmin_init")[0] == 2  # calls 1 and 2
    idx.add(x[:5])  # new rows: the last step no longer describes these points
    c = steps[3]
    x2 = np.concatenate([x, x[:5]])
    r = vs.kmeans_step(idx, c, 1, u)
    ar, cr, _, objr = _kmeans_oracle_step(x2, c, u)
    assert np.array_equal(r[0], ar) and r[3] == objr
    assert idx.prof_get("kmin_init")[0] == 2
    idx.close()


def test_kmeans_second_step_grouped_order(vs):
    """The pick of a second step walks the points grouped by the first
    step's clusters (a permutation): the same assignments, objective and
    centroids as the oracle's, and as walking them in index order."""
    x, _ = syn.gaussian_mixture(30_000, 256, 512, 0.1, 45)
    cen = x[syn.seeded_subset(30_000, 2048, 45)].copy()
    u = syn.rng(46, 0).random(2048 * 256)
    pts = vs.GpuIndexFlat.l2(256, storage="f32")
    pts.add(x)
    _, cen1, _, _ = vs.kmeans_step(pts, cen, 1, u)
    a2, c2, n2, o2 = vs.kmeans_step(pts, cen1, 1, u)
    pts.set_option("pick_order", 0)
    a3, c3, n3, o3 = vs.kmeans_step(pts, cen1, 1, u)
    pts.close()
    assert np.array_equal(a2, a3) and o2 == o3
    assert np.array_equal(c2.view(np.uint32), c3.view(np.uint32)) and np.array_equal(n2, n3)
    ar, _, objr = oracle.kmeans_assign(x, cen1, NT)
    assert np.array_equal(a2, ar) and o2 == objr


def test_kmeans_assign_order_matches_index_order(vs):
    """From the second step on the assign scan walks the points grouped by
    the last step's clusters (option assign_order, the default), their
    lists and counts still indexed by point: three chained steps on 30,000
    points (ending inside a 256-point block) give the same assignments,
    objective and centroids as index order, and the oracle's."""
    x, _ = syn.gaussian_mixture(30_000, 256, 1024, 0.1, 52)
    cen = x[syn.seeded_subset(30_000, 4096, 52)].copy()
    u = syn.rng(53, 0).random(4096 * 256)
    a = vs.GpuIndexFlat.l2(256, storage="f32")
    b = vs.GpuIndexFlat.l2(256, storage="f32")
    a.add(x)
    b.add(x)
    b.set_option("assign_order", 0)
    ca = cb = cen
    for step in range(3):
        ra = vs.kmeans_step(a, ca, 1, u)
        rb = vs.kmeans_step(b, cb, 1, u)
        ar, cr, cntr, objr = _kmeans_oracle_step(x, ca, u)
        assert np.array_equal(ra[0], ar), f"step {step}: {np.sum(ra[0] != ar)} assignments differ"
        assert ra[3] == objr and np.array_equal(ra[2], cntr)
        assert np.array_equal(ra[1].view(np.uint32), cr.view(np.uint32))
        assert np.array_equal(ra[0], rb[0]) and ra[3] == rb[3]
        assert np.array_equal(ra[1].view(np.uint32), rb[1].view(np.uint32))
        ca, cb = ra[1], rb[1]
    assert a.prof_get("assign_order")[0] == 2 and b.prof_get("assign_order")[0] == 0
    a.close()
    b.close()
