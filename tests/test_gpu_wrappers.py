"""The reference's wrapper indexes over the GPU flat index
(index_id_map.dart, index_pre_transform.dart, index_refine_flat.dart,
index_shards.dart), each against the same semantics restated on the CPU
oracle (IndexFlat.search, index_flat.dart:62-97)."""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def data(n=4000, d=32, nq=25, seed=3):
    g = syn.rng(seed, 0)
    return (g.standard_normal((n, d)).astype(np.float32),
            g.standard_normal((nq, d)).astype(np.float32))


@pytest.mark.parametrize("metric", [0, 1])
def test_id_map(vs, metric):
    x, q = data()
    g = syn.rng(4, 1)
    ext = g.choice(np.arange(-(1 << 31), (1 << 31) - 1, 1000, dtype=np.int64), size=len(x),
                   replace=False)
    m = vs.IndexIDMap(vs.GpuIndexFlat(32, vs.Metric(metric), storage="f32"))
    m.add_with_ids(x, ext)
    r = m.search(q, 8)
    Dr, Ir = oracle.flat_search(x, q, 8, metric, NT)
    assert_knn_parity(r.distances, r.ids, Dr, ext[Ir].astype(np.int32), metric)
    with pytest.raises(ValueError, match="does not fit in int32"):
        m.add_with_ids(x[:1], [1 << 31])
    # removeIds by external id compacts both sides (index_id_map.dart:112-134)
    gone = set(int(e) for e in ext[Ir[:, 0]])
    assert m.remove_ids(gone | {12345}) == len(gone)
    keep = np.array([e not in gone for e in ext])
    r = m.search(q, 8)
    Dr, Ir = oracle.flat_search(x[keep], q, 8, metric, NT)
    assert_knn_parity(r.distances, r.ids, Dr, ext[keep][Ir].astype(np.int32), metric)
    # range search ids are external too
    rr = m.range_search(q[:3], float(Dr[0, 4]))
    assert set(rr.ids.tolist()) <= set(ext[keep].astype(np.int32).tolist())
    m.inner.close()


def test_pre_transform_l2norm(vs):
    x, q = data(d=48)
    p = vs.IndexPreTransform([vs.L2NormTransform(48)], vs.GpuIndexFlat.ip(48, storage="f32"))
    p.add(x)
    r = p.search(q, 10)
    xn, qn = syn.l2_normalize(x), syn.l2_normalize(q)
    Dr, Ir = oracle.flat_search(xn, qn, 10, 1, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 1)
    with pytest.raises(ValueError):
        vs.IndexPreTransform([vs.L2NormTransform(40)], vs.GpuIndexFlat.ip(48))
    p.inner.close()


@pytest.mark.parametrize("metric", [0, 1])
def test_refine_flat_over_ivf(vs, metric):
    """The exact re-rank of the base index's k * kFactor candidates, on the
    GPU, equals the oracle re-ranking the same candidates."""
    x, q = data(n=6000, d=24)
    ivf = vs.IndexIVFFlat(24, 16, metric=vs.Metric(metric), nprobe=2, kmeans_iters=4)
    ref = vs.IndexRefineFlat(ivf, k_factor=3)
    ref.train(x[:2000])
    ref.add(x)
    r = ref.search(q, 7)
    cand = ivf.search(q, 21).ids
    for qi in range(len(q)):
        c = cand[qi][cand[qi] >= 0].astype(np.int64)
        Dr, Ir = oracle.flat_search(x[c], q[qi:qi + 1], 7, metric, 1)
        Ir = np.where(Ir >= 0, c[np.maximum(Ir, 0)], -1).astype(np.int32)
        assert_knn_parity(r.distances[qi:qi + 1], r.ids[qi:qi + 1], Dr, Ir, metric)
    ref.close()
    ivf.close()


@pytest.mark.parametrize("metric", [0, 1])
def test_shards_equal_flat(vs, metric):
    x, q = data(n=5003)
    sh = vs.IndexShards([vs.GpuIndexFlat(32, vs.Metric(metric), storage="f32") for _ in range(3)])
    sh.add(x[:2000])
    sh.add(x[2000:])  # external ids continue across adds (id % nshards picks the shard)
    assert sh.ntotal == len(x) and [s.ntotal for s in sh.shards] == [1668, 1668, 1667]
    r = sh.search(q, 12)
    Dr, Ir = oracle.flat_search(x, q, 12, metric, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, metric)
    for s in sh.shards:
        s.close()


def test_shards_prepopulated(vs):
    """Shards that already hold rows: ntotal starts at their sum (the
    reference's constructor folds it), so later adds continue the external id
    sequence and its round-robin dealing (index_shards.dart constructor, add)."""
    x, q = data(n=3000)
    a, b = (vs.GpuIndexFlat(32, vs.Metric.l2, storage="f32") for _ in range(2))
    # external ids 0..999 dealt round-robin by hand: even ids in a, odd in b
    a.add(x[0:1000:2])
    b.add(x[1:1000:2])
    sh = vs.IndexShards([a, b])
    assert sh.ntotal == 1000
    sh.add(x[1000:])
    assert sh.ntotal == 3000 and a.ntotal == 1500 and b.ntotal == 1500
    r = sh.search(q, 10)
    Dr, Ir = oracle.flat_search(x, q, 10, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0)
    a.close()
    b.close()


def test_id_map_duplicate_external_ids(vs):
    """A duplicated external id resolves to its last internal offset, as the
    reference's reverse map built in offset order does (index_id_map.dart
    internalOf); ids never added give -1."""
    x, _ = data(n=6)
    m = vs.IndexIDMap(vs.GpuIndexFlat(32, vs.Metric.l2, storage="f32"))
    m.add_with_ids(x, [7, 3, 7, 9, 3, 5])
    assert [m.internal_of(e) for e in (7, 3, 9, 5, 11)] == [2, 4, 3, 5, -1]
    assert m.id_of(0) == 7 and m.id_of(4) == 3
    m.inner.close()
