"""The IVF coarse path on the GPU flat scan (index_ivf_flat.dart:84-171) and
the k-means it trains with (kmeans.dart:48-140), against restatements on the
CPU oracle (IndexFlat.search, the k-means assign / update steps) driven by
the same random generator."""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def blobs(n, d, k=12, std=0.08, seed=1):
    g = syn.rng(seed, 7)
    centers = g.uniform(-1, 1, size=(k, d)).astype(np.float32)
    lab = g.integers(0, k, size=n)
    return (centers[lab] + g.normal(0, std, size=(n, d))).astype(np.float32)


def l2sq_to(x, c):
    """fp32 of the reference's fp64 squared distance of every row to c."""
    _, best, _ = oracle.kmeans_assign(x, c[None, :], NT)
    return best.astype(np.float32)


def kmeanspp_restated(x, k, rng):
    """kmeans.dart:48-85 on the oracle's arithmetic, scalar loops."""
    n, d = x.shape
    cen = np.empty((k, d), np.float32)
    cen[0] = x[int(rng.integers(n))]
    closest = l2sq_to(x, cen[0])
    for c in range(1, k):
        s = 0.0
        for v in closest:
            s += float(v)
        if s <= 0:
            cen[c] = x[int(rng.integers(n))]
        else:
            target = rng.random() * s
            acc, pick = 0.0, n - 1
            for i, v in enumerate(closest):
                acc += float(v)
                if acc >= target:
                    pick = i
                    break
            cen[c] = x[pick]
        dsq = l2sq_to(x, cen[c])
        closest = np.where(dsq < closest, dsq, closest)
    return cen


def test_kmeanspp_matches_restatement(vs):
    from vector_store.kmeans import kmeans_pp_init

    x = blobs(1500, 16, seed=3)
    pts = vs.GpuIndexFlat.l2(16, storage="f32")
    pts.add(x)
    got = kmeans_pp_init(pts, x, 24, np.random.Generator(np.random.Philox(99)))
    pts.close()
    want = kmeanspp_restated(x, 24, np.random.Generator(np.random.Philox(99)))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_kmeans_train_matches_oracle_iterations(vs):
    """Kmeans.train: init, then assign / update per iteration with jitter
    drawn only for empty clusters; bit-identical centroids, assignments and
    objective, and a non-increasing objective (vector_store_test.dart:91-111)."""
    x = blobs(2000, 8, k=6, seed=5)
    k, niter, seed = 40, 6, 1234  # more clusters than blobs: empty clusters occur
    res = vs.Kmeans(8, k, niter=niter, seed=seed).train(x)
    rng = np.random.Generator(np.random.Philox(seed))
    cen = kmeanspp_restated(x, k, rng)
    objs = []
    for _ in range(niter):
        a, _, obj = oracle.kmeans_assign(x, cen, NT)
        state = rng.bit_generator.state
        offer = rng.random(k * 8)
        cen, counts, used = oracle.kmeans_update(x, a, cen, 1, offer)
        rng.bit_generator.state = state
        rng.random(used)
        objs.append(obj)
    assert np.array_equal(res.assignments, a)
    assert np.array_equal(res.centroids.view(np.uint32), cen.view(np.uint32))
    assert res.objective == objs[-1]
    assert all(b <= a0 * (1 + 1e-12) for a0, b in zip(objs, objs[1:]))


@pytest.mark.parametrize("metric", [0, 1])
def test_ivf_add_and_search_match_restatement(vs, metric):
    d, nlist, nprobe, k = 24, 16, 3, 10
    x = blobs(6000, d, k=nlist, seed=11)
    q = blobs(40, d, k=nlist, seed=12)
    ivf = vs.IndexIVFFlat(d, nlist, metric=vs.Metric(metric), nprobe=nprobe, kmeans_iters=5)
    ivf.train(x[:3000])
    ivf.add(x)
    cen = ivf.quantizer.reconstruct_n(0, nlist)
    # assignment: the quantizer's k = 1 search (index_ivf_flat.dart:117-127)
    _, cell = oracle.flat_search(cen, x, 1, metric, NT)
    lists = [[] for _ in range(nlist)]
    for i, c in enumerate(cell[:, 0].tolist()):
        lists[c].append(i)
    assert ivf.inv_lists == lists
    # search: nprobe cells, exact scan of their lists (:132-171)
    r = ivf.search(q, k)
    _, probes = oracle.flat_search(cen, q, nprobe, metric, NT)
    for qi in range(len(q)):
        cand = np.array(sorted(i for c in probes[qi] if c >= 0 for i in lists[c]), np.int64)
        Dr, Ir = oracle.flat_search(x[cand], q[qi:qi + 1], k, metric, 1)
        Ir = np.where(Ir >= 0, cand[np.maximum(Ir, 0)], -1).astype(np.int32)
        assert_knn_parity(r.distances[qi:qi + 1], r.ids[qi:qi + 1], Dr, Ir, metric)
    # every cell probed: the flat result (recall 1.0, bench test at nprobe == nlist)
    ivf.nprobe = nlist
    r = ivf.search(q, k)
    Dr, Ir = oracle.flat_search(x, q, k, metric, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, metric)
    ivf.close()


def test_subset_search_edges(vs):
    x = blobs(500, 8, seed=2)
    g = vs.GpuIndexFlat.l2(8, storage="f32")
    g.add(x)
    ids = np.arange(0, 500, 7, dtype=np.int32)  # 72 ids
    q = x[:3]
    # query 0: two segments, query 1: one empty and one short, query 2: nothing
    off = np.array([[0, 30], [0, 60], [0, 0]], np.int64)
    ln = np.array([[30, 42], [0, 5], [0, 0]], np.int64)
    r = g.search_subsets(q, 6, ids, off, ln)
    Dr, Ir = oracle.flat_search(x[ids], q[:1], 6, 0)
    assert np.array_equal(r.ids[0], ids[Ir[0]]) and np.array_equal(r.distances[0], Dr[0])
    assert list(r.ids[1, :5]) == sorted(ids[60:65].tolist(), key=lambda i: float(
        np.sum((x[i].astype(np.float64) - q[1]) ** 2))) and r.ids[1, 5] == -1
    assert np.all(r.ids[2] == -1) and np.all(np.isinf(r.distances[2]))
    with pytest.raises(ValueError):
        g.search_subsets(q, 6, np.array([0, 9999], np.int32), off[:, :1] * 0,
                         np.array([[2], [0], [0]], np.int64))
    g.close()


@pytest.mark.parametrize("metric", [0, 1])
def test_subset_search_large_k(vs, metric):
    """k beyond the list path (600 > 409): each query's subset rows scored
    in fp64 and sorted by (fp32 score, id) -- the oracle's top-k over those
    rows, sentinels past the subset's size (query 1 names 250 rows, query 2
    none) -- and the list path's k = 400 answers are its first 400."""
    x = blobs(5000, 24, seed=4)
    g = vs.GpuIndexFlat(24, vs.Metric(metric), storage="f32")
    g.add(x)
    ids = syn.rng(5, 0).permutation(5000)[:3000].astype(np.int32)
    q = (x[[7, 11, 13]] + 0.01).astype(np.float32)
    off = np.array([[0, 2000], [100, 0], [0, 0]], np.int64)
    ln = np.array([[1500, 800], [250, 0], [0, 0]], np.int64)
    k = 600
    r = g.search_subsets(q, k, ids, off, ln)
    r4 = g.search_subsets(q, 400, ids, off, ln)
    g.close()
    for i in range(3):
        rows = np.concatenate([ids[o:o + n] for o, n in zip(off[i], ln[i])]).astype(np.int64)
        if len(rows) == 0:
            assert np.all(r.ids[i] == -1)
            assert np.all(np.isinf(r.distances[i]))
            continue
        Dr, Ir = oracle.flat_search(x[rows], q[i:i + 1], k, metric)
        Ir = np.where(Ir >= 0, rows[np.maximum(Ir, 0)], -1).astype(np.int32)
        assert_knn_parity(r.distances[i:i + 1], r.ids[i:i + 1], Dr, Ir, metric)
        assert (r.ids[i] >= 0).sum() == min(k, len(rows))
    assert np.array_equal(r.ids[:, :400], r4.ids) and np.array_equal(r.distances[:, :400], r4.distances)
