"""GPU k-NN search parity against the CPU oracle (restating IndexFlat.search,
lib/core/vector_store/index_flat.dart:62-97) on identical seeded inputs."""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def blobs(n, d, k=8, std=0.05, seed=1):
    """Clustered data shaped like the reference's _sampleBlobs (vector_store_test.dart:9-35)."""
    g = syn.rng(seed, 7)
    centers = g.uniform(-1, 1, size=(k, d)).astype(np.float32)
    lab = g.integers(0, k, size=n)
    noise = (g.random((n, d)) + g.random((n, d)) - 1.0) * std
    return (centers[lab] + noise).astype(np.float32)


def run(vs, xb, xq, k, metric, storage="f32", qdtype=None):
    idx = vs.GpuIndexFlat(xb.shape[1], vs.Metric(metric), storage=storage)
    idx.add(xb)
    q = xq if qdtype is None else qdtype(xq)
    r = idx.search(q, k)
    idx.close()
    return r.distances, r.ids


@pytest.mark.parametrize("metric", [0, 1])
def test_reference_fixture_shape(vs, metric):
    """d=16, n=400, nq=20, k=5 (vector_store_test.dart:51-54)."""
    xb, xq = blobs(400, 16, seed=1), blobs(20, 16, seed=2)
    D, I = run(vs, xb, xq, 5, metric)
    Dr, Ir = oracle.flat_search(xb, xq, 5, metric, NT)
    assert_knn_parity(D, I, Dr, Ir, metric)


def test_self_match_l2_and_ip(vs):
    """vector_store_test.dart:66-89: L2 self-search gives id i at distance 0;
    IP top score >= |x|^2 - 1e-4."""
    xb = blobs(400, 16, seed=1)
    D, I = run(vs, xb, xb[:3], 1, 0)
    assert list(I[:, 0]) == [0, 1, 2]
    assert np.all(np.abs(D[:, 0]) <= 1e-5)
    D, I = run(vs, xb, xb[:3], 1, 1)
    self_ip = (xb[:3].astype(np.float64) ** 2).sum(1)
    assert np.all(D[:, 0] >= self_ip - 1e-4)


@pytest.mark.parametrize("metric", [0, 1])
def test_gpu_threshold_size(vs, metric):
    """n=4096, d=16 (vector_store_test.dart:3565-3605), now at full parity
    instead of the reference's 1e-2 tolerance."""
    xb, xq = blobs(4096, 16, seed=7), blobs(20, 16, seed=8)
    D, I = run(vs, xb, xq, 5, metric)
    Dr, Ir = oracle.flat_search(xb, xq, 5, metric, NT)
    assert_knn_parity(D, I, Dr, Ir, metric)


def test_config1_full(vs):
    """10k x 384 unit N(0,1) IP, 100 queries, k=10."""
    xb = syn.normal_unit(10_000, 384, 1234, 0)
    xq = syn.normal_unit(100, 384, 1234, 1)
    D, I = run(vs, xb, xq, 10, 1)
    Dr, Ir = oracle.flat_search(xb, xq, 10, 1, NT)
    assert_knn_parity(D, I, Dr, Ir, 1)


@pytest.mark.parametrize("nq", [1, 64, 200])
def test_config2_slice_exact(vs, nq):
    """configs[1] shape on a 100k-row slice: integers 0..255, L2, k=100.
    Integer sums stay below 2^24, so distances are exact integers and equal
    bit for bit; ids are compared per tie group (ties are frequent)."""
    xb = syn.int_grid(100_000, 128, 1234, 0)
    xq = syn.int_grid(nq, 128, 1234, 1)
    idx = vs.GpuIndexFlat(128, vs.Metric.l2, storage="auto")
    idx.add(xb)
    assert idx.storage == "bf16"  # lossless: every value is a bf16 value
    r = idx.search(xq, 100)
    Dr, Ir = oracle.flat_search(xb, xq, 100, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)
    assert np.all(r.distances == np.round(r.distances))


@pytest.mark.parametrize("nq", [1, 7, 64, 300])
def test_bf16_storage_ip(vs, nq):
    """configs[2] arithmetic on a 60k x 768 slice: bf16 unit vectors, IP, k=10;
    the oracle is fed the same bf16 values upcast to fp32."""
    xb16 = syn.to_bf16_bits(syn.normal_unit(60_000, 768, 99, 0))
    xq16 = syn.to_bf16_bits(syn.normal_unit(nq, 768, 99, 1))
    idx = vs.GpuIndexFlat(768, vs.Metric.innerProduct, storage="bf16")
    idx.add(xb16)
    r = idx.search(xq16, 10)
    Dr, Ir = oracle.flat_search(syn.bf16_bits_to_f32(xb16), syn.bf16_bits_to_f32(xq16), 10, 1, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 1, rtol=1e-3)


def test_eight_wave_streaming_scan(vs, opts):
    """Regression test of the 8-wave streaming scan (option scan_nw8), whose
    LDS id area once started at the 4-wave offset: the batch-64 shape of
    test_bf16_storage_ip, where it runs, against the oracle."""
    opts(scan_nw8=1)
    xb16 = syn.to_bf16_bits(syn.normal_unit(60_000, 768, 99, 0))
    xq16 = syn.to_bf16_bits(syn.normal_unit(64, 768, 99, 1))
    idx = vs.GpuIndexFlat(768, vs.Metric.innerProduct, storage="bf16")
    idx.add(xb16)
    idx.prof_reset()
    r = idx.search(xq16, 10)
    n8 = idx.prof_get("streamed8")[0]
    idx.close()
    assert n8 >= 1, "the 8-wave scan did not run"
    Dr, Ir = oracle.flat_search(syn.bf16_bits_to_f32(xb16), syn.bf16_bits_to_f32(xq16), 10, 1, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 1, rtol=1e-3)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 1, rtol=1e-3)


def test_bf16_storage_fp32_queries(vs):
    """bf16 rows, fp32 queries (two query planes): the oracle sees the stored
    bf16 values and the fp32 queries as given."""
    xb16 = syn.to_bf16_bits(syn.normal_unit(20_000, 256, 5, 0))
    xq = syn.normal_unit(40, 256, 5, 1)
    idx = vs.GpuIndexFlat(256, vs.Metric.l2, storage="bf16")
    idx.add(xb16)
    r = idx.search(xq, 10)
    Dr, Ir = oracle.flat_search(syn.bf16_bits_to_f32(xb16), xq, 10, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0, rtol=1e-5)


@pytest.mark.parametrize("d", [1, 3, 17, 100, 130, 512])
@pytest.mark.parametrize("metric", [0, 1])
def test_ragged_dims(vs, d, metric):
    xb = syn.rng(3, d).standard_normal((3000, d)).astype(np.float32)
    xq = syn.rng(4, d).standard_normal((33, d)).astype(np.float32)
    D, I = run(vs, xb, xq, 7, metric)
    Dr, Ir = oracle.flat_search(xb, xq, 7, metric, NT)
    assert_knn_parity(D, I, Dr, Ir, metric)


def test_k_larger_than_ntotal_gives_sentinels(vs):
    """index.dart:306-313: missing slots are +inf / -inf with id -1."""
    xb = blobs(5, 16)
    for metric, sent in ((0, np.inf), (1, -np.inf)):
        D, I = run(vs, xb, blobs(3, 16, seed=5), 8, metric)
        Dr, Ir = oracle.flat_search(xb, blobs(3, 16, seed=5), 8, metric, 1)
        assert np.all(I[:, 5:] == -1) and np.all(D[:, 5:] == sent)
        assert_knn_parity(D, I, Dr, Ir, metric)


def test_duplicates_tie_to_lowest_ids(vs):
    """Identical vectors tie exactly; strict acceptance keeps the first ids."""
    row = syn.rng(1, 1).standard_normal(32).astype(np.float32)
    xb = np.tile(row, (500, 1))
    D, I = run(vs, xb, row[None, :], 10, 0)
    assert sorted(I[0].tolist()) == list(range(10))
    assert np.all(D[0] == 0.0)


def test_large_k_and_many_queries(vs):
    xb = syn.rng(9, 0).standard_normal((20_000, 48)).astype(np.float32)
    xq = syn.rng(9, 1).standard_normal((150, 48)).astype(np.float32)
    for k in (1, 33, 256, 400):
        D, I = run(vs, xb, xq, k, 0)
        Dr, Ir = oracle.flat_search(xb, xq, k, 0, NT)
        assert_knn_parity(D, I, Dr, Ir, 0)


def test_edge_cases(vs):
    idx = vs.GpuIndexFlat.l2(8)
    r = idx.search(np.zeros((0, 8), np.float32), 3)  # nq = 0
    assert r.nq == 0
    r = idx.search(np.ones((2, 8), np.float32), 3)  # empty index
    assert np.all(r.ids == -1) and np.all(np.isinf(r.distances))
    idx.add(np.ones((4, 8), np.float32))
    with pytest.raises(ValueError):
        idx.search(np.ones((2, 8), np.float32), 0)  # TopK(0) throws in the reference
    with pytest.raises(ValueError):
        idx.search(np.ones((2, 7), np.float32), 3)  # query length != d
    with pytest.raises(ValueError):
        idx.add(np.ones((2, 9), np.float32))
    bad = np.ones((2, 8), np.float32)
    bad[1, 3] = np.nan
    with pytest.raises(vs.VsError):
        idx.add(bad)
    with pytest.raises(vs.VsError):
        idx.search(bad, 2)
    assert idx.ntotal == 4  # failed add left nothing behind
    r = idx.search(np.ones((1, 8), np.float32), 1000)  # any k, as TopK accepts it
    assert np.all(r.ids[0, :4] >= 0) and np.all(r.ids[0, 4:] == -1)
    assert np.all(np.isinf(r.distances[0, 4:])) and np.all(r.distances[0, :4] == 0.0)
    idx.close()


@pytest.mark.parametrize("nq,bad_bits", [(1, 0x7FC0), (64, 0x7F80), (300, 0xFF80)])
def test_nonfinite_bf16_queries(vs, nq, bad_bits):
    """bf16 queries take one MFMA plane whatever their values, so the search
    reads their flags together with its results instead of waiting for them
    first; meanwhile a row holding NaN or an infinity is searched as a unit
    vector.  The call still fails with VS_ERR_NONFINITE, on the host and the
    device entry points, and the next search is exact again."""
    xb = syn.int_grid(300_000, 64, 13, 0)
    q16 = syn.to_bf16_bits(syn.int_grid(nq, 64, 13, 3))
    bad = q16.copy()
    bad[nq // 2, 5] = bad_bits
    idx = vs.GpuIndexFlat(64, vs.Metric.innerProduct, storage="auto")
    idx.add(xb)
    with pytest.raises(vs.VsError) as e:
        idx.search(bad, 10)
    assert e.value.code == vs._native.VS_ERR_NONFINITE
    qd = vs._native.DeviceBuffer(bad.nbytes)
    qd.upload(bad)
    Dd = vs._native.DeviceBuffer(nq * 10 * 4)
    Id = vs._native.DeviceBuffer(nq * 10 * 4)
    with pytest.raises(vs.VsError) as e:
        idx.search_device(qd, nq, 10, Dd, Id, dtype=vs._native.VS_DTYPE_BF16)
    assert e.value.code == vs._native.VS_ERR_NONFINITE
    r = idx.search(q16, 10)
    idx.close()
    for b in (qd, Dd, Id):
        b.free()
    xq = syn.bf16_bits_to_f32(q16)
    Dr, Ir = oracle.flat_search(xb, xq, 10, 1, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 1, rtol=0.0, atol=0.0, xb=xb, xq=xq)


def test_add_after_search_and_wrap(vs):
    """vector_store_test.dart:3607-3637: a vector added after a search is found
    at id old_ntotal; wrap() keeps the ranking."""
    xb = blobs(400, 16)
    g = vs.GpuIndexFlat.l2(16)
    g.add(xb)
    g.warmup()
    g.search(xb[:2], 3)
    new = np.full((1, 16), 99.0, np.float32)
    old = g.ntotal
    g.add(new)
    assert g.ntotal == old + 1
    r = g.search(new, 1)
    assert r.ids[0, 0] == old and abs(r.distances[0, 0]) <= 1e-3
    w = vs.GpuIndexFlat.wrap(g)
    assert w.d == 16 and w.ntotal == g.ntotal
    q = blobs(2, 16, seed=2)
    assert np.array_equal(w.search(q, 1).ids, g.search(q, 1).ids)


def test_auto_storage_widens(vs):
    """AUTO keeps bf16 while lossless, switches to fp32 at the first inexact add."""
    a = syn.int_grid(3000, 64, 1, 0)
    b = syn.rng(2, 0).standard_normal((2000, 64)).astype(np.float32)
    idx = vs.GpuIndexFlat.l2(64, storage="auto")
    idx.add(a)
    assert idx.storage == "bf16"
    idx.add(b)
    assert idx.storage == "f32"
    xb = np.concatenate([a, b])
    assert np.array_equal(idx.reconstruct_n(0, 5000), xb)
    xq = syn.rng(3, 0).standard_normal((20, 64)).astype(np.float32) * 50
    r = idx.search(xq, 10)
    Dr, Ir = oracle.flat_search(xb, xq, 10, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0)


def test_remove_ids(vs):
    """vector_store_test.dart:384-403: remove every third id, compact, renumber."""
    xb = blobs(400, 16)
    g = vs.GpuIndexFlat.l2(16)
    g.add(xb)
    drop = set(range(0, 400, 3))
    assert g.remove_ids(drop | {1000, -5}) == len(drop)
    kept = np.array([xb[i] for i in range(400) if i not in drop])
    assert g.ntotal == len(kept)
    assert np.array_equal(g.reconstruct_n(0, len(kept)), kept)
    r = g.search(kept[:5], 1)
    assert np.all(np.abs(r.distances[:, 0]) <= 1e-5) and list(r.ids[:, 0]) == [0, 1, 2, 3, 4]
    Dr, Ir = oracle.flat_search(kept, blobs(10, 16, seed=3), 4, 0, 1)
    r = g.search(blobs(10, 16, seed=3), 4)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0)


def test_faisdart_fixtures(vs):
    """The reference's two FAISDART IndexFlatIP fixtures (data/*/index.bin):
    each stored vector's top-1 is itself; full parity with the oracle."""
    import os

    from vector_store import io as vio

    for name in ("docs_index.bin", "qa_index.bin"):
        hdr, xb = vio.read_faisdart_flat(os.path.join(os.path.dirname(__file__), "golden", name))
        assert hdr["metric"] == 1 and hdr["d"] == 384 and hdr["ntotal"] == 20
        g = vs.GpuIndexFlat.ip(384)
        g.add(xb)
        r = g.search(xb, 5)
        assert list(r.ids[:, 0]) == list(range(20))
        Dr, Ir = oracle.flat_search(xb, xb, 5, 1, 1)
        assert_knn_parity(r.distances, r.ids, Dr, Ir, 1)


@pytest.mark.parametrize("k", [10, 50, 100])
def test_short_lists_are_verified(vs, opts, k):
    """Per-wave lists may keep fewer than the merged candidates; the merge
    proves no list dropped a winner or re-runs the query with full lists.
    Rows sorted by distance to query 0 put all its winners in one list, and a
    forced 4-entry list keep makes the proof fail: the re-run must still
    give the oracle's answer."""
    g = syn.rng(21, 0)
    xq = g.standard_normal((3, 32)).astype(np.float32)
    xb = g.standard_normal((8000, 32)).astype(np.float32)
    xb = xb[np.argsort(((xb.astype(np.float64) - xq[0]) ** 2).sum(1), kind="stable")]
    opts(scan_kkw=4)
    idx = vs.GpuIndexFlat.l2(32, storage="f32")
    idx.add(xb)
    r = idx.search(xq, k)
    reruns, _ = idx.prof_get("fallback")
    idx.close()
    Dr, Ir = oracle.flat_search(xb, xq, k, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0)
    assert reruns >= 1


@pytest.mark.parametrize("nq,k,metric", [(1, 10, 1), (37, 10, 0), (64, 100, 0), (16, 100, 1)])
def test_small_batch_prepass(vs, nq, k, metric):
    """Small batches over 300,000 rows plan many short lists, so a pre-pass
    over a sample of the rows seeds every query's shared threshold before
    the full scan.  Integer data (exact distances): the result equals the
    oracle's, and the distances equal those of a search without the
    pre-pass (option prepass = 0)."""
    xb = syn.int_grid(300_000, 64, 8, 0)
    xq = syn.int_grid(nq, 64, 8, 1)
    idx = vs.GpuIndexFlat(64, vs.Metric(metric), storage="auto")
    idx.add(xb)
    r1 = idx.search(xq, k)
    npre, _ = idx.prof_get("prepass_scans")
    idx.set_option("prepass", 0)
    r0 = idx.search(xq, k)
    npre0, _ = idx.prof_get("prepass_scans")
    idx.close()
    assert npre >= 1 and npre0 == npre
    Dr, Ir = oracle.flat_search(xb, xq, k, metric, NT)
    assert_knn_parity(r1.distances, r1.ids, Dr, Ir, metric, rtol=0.0, atol=0.0, xb=xb, xq=xq)
    assert np.array_equal(r1.distances, r0.distances)


@pytest.mark.parametrize("nq,k,metric", [(512, 100, 0), (300, 10, 1), (1024, 1, 0)])
def test_large_batch_estimated_threshold(vs, nq, k, metric):
    """Large batches over 2^18+ rows start every query's threshold from an
    estimate taken on a sample of the rows (a rank of the sample chosen so
    that kk_final rows of the full scan very likely lie below it).  Integer
    data: the result equals the oracle's and a search without the estimate
    (option guess = 0), and no query needed the exact re-search."""
    xb = syn.int_grid(300_000, 32, 11, 0)
    xq = syn.int_grid(nq, 32, 11, 1)
    idx = vs.GpuIndexFlat(32, vs.Metric(metric), storage="auto")
    idx.add(xb)
    idx.prof_reset()
    r1 = idx.search(xq, k)
    ng, _ = idx.prof_get("guess_scans")
    nfb, _ = idx.prof_get("fallback")
    idx.set_option("guess", 0)
    r0 = idx.search(xq, k)
    ng0, _ = idx.prof_get("guess_scans")
    idx.close()
    assert ng == 1 and ng0 == 1 and nfb == 0
    sub = np.arange(0, nq, 7)
    Dr, Ir = oracle.flat_search(xb, xq[sub], k, metric, NT)
    assert_knn_parity(r1.distances[sub], r1.ids[sub], Dr, Ir, metric, rtol=0.0, atol=0.0,
                      xb=xb, xq=xq[sub])
    assert np.array_equal(r1.distances, r0.distances)


@pytest.mark.parametrize("nq,k,metric", [(5, 100, 0), (64, 10, 1), (300, 100, 1)])
def test_merge_chunks_per_pass(vs, nq, k, metric):
    """The merge reads 1, 2, 4 or 8 chunks of 1024 list entries per pass
    (option merge_mu; by default more when the batch is small).  Over
    300,000 integer rows -- a threshold pre-pass or estimate, thousands of
    lists per query, buffer cuts -- every setting gives the oracle's result."""
    xb = syn.int_grid(300_000, 64, 13, 0)
    xq = syn.int_grid(nq, 64, 13, 1)
    idx = vs.GpuIndexFlat(64, vs.Metric(metric), storage="auto")
    idx.add(xb)
    res = {}
    for mu in (1, 2, 4, 8):
        idx.set_option("merge_mu", mu)
        res[mu] = idx.search(xq, k)
    idx.close()
    sub = np.arange(0, nq, 3)
    Dr, Ir = oracle.flat_search(xb, xq[sub], k, metric, NT)
    for mu, r in res.items():
        assert_knn_parity(r.distances[sub], r.ids[sub], Dr, Ir, metric, rtol=0.0, atol=0.0,
                          xb=xb, xq=xq[sub])
        assert np.array_equal(r.distances, res[1].distances), mu


@pytest.mark.parametrize("nq,k,metric", [(1, 10, 1), (5, 100, 0), (64, 10, 1), (40, 400, 0)])
def test_split_merge(vs, nq, k, metric):
    """A batch with fewer queries than half the CUs' worth of workgroups
    splits each query's list entries over several merge workgroups (option
    merge_g; 0 plans it), each keeping its slice's kk_final best pairs, and
    a second pass merges those -- for the threshold seeding and for the
    final merge.  Integer rows with many tied distances: every split count
    gives the one-workgroup merge's result, equal to the oracle's."""
    xb = syn.int_grid(300_000, 64, 13, 0)
    xq = syn.int_grid(nq, 64, 13, 2)
    idx = vs.GpuIndexFlat(64, vs.Metric(metric), storage="auto")
    idx.add(xb)
    res, nsplit = {}, {}
    for g in (1, 2, 7, 64, 0):
        idx.set_option("merge_g", g)
        idx.prof_reset()
        res[g] = idx.search(xq, k)
        nsplit[g] = idx.prof_get("split_merges")[0]
    idx.close()
    assert nsplit[1] == 0 and nsplit[2] == 2 and nsplit[7] == 2 and nsplit[64] == 2
    assert nsplit[0] == 2  # planned: these batches leave most CUs idle
    Dr, Ir = oracle.flat_search(xb, xq, k, metric, NT)
    for g, r in res.items():
        assert_knn_parity(r.distances, r.ids, Dr, Ir, metric, rtol=0.0, atol=0.0, xb=xb, xq=xq)
        assert np.array_equal(r.distances, res[1].distances), g
        assert np.array_equal(r.ids, res[1].ids), g


def test_estimated_threshold_too_tight_falls_back(vs):
    """A sample that is not representative: the first 1/16 of the rows holds
    64 near copies of every query, the rest lies far away.  The estimate
    (the 24th sample value at k = 100) then leaves only about 64 rows of the
    full scan below it, fewer than the 128 the merge needs, so every query
    is searched again exactly -- and the result still equals the oracle's."""
    n, d, nq, k = 1 << 18, 16, 256, 100
    g = syn.rng(5, 3)
    xq = g.integers(0, 64, size=(nq, d)).astype(np.float32)
    xb = g.integers(128, 256, size=(n, d)).astype(np.float32)
    near = n // 16
    xb[:near] = xq[np.arange(near) % nq] + g.integers(0, 3, size=(near, d)).astype(np.float32)
    idx = vs.GpuIndexFlat(d, vs.Metric(0), storage="auto")
    idx.add(xb)
    idx.prof_reset()
    r = idx.search(xq, k)
    ng, _ = idx.prof_get("guess_scans")
    nfb, _ = idx.prof_get("fallback")
    idx.close()
    assert ng == 1 and nfb == nq
    sub = np.arange(0, nq, 5)
    Dr, Ir = oracle.flat_search(xb, xq[sub], k, 0, NT)
    assert_knn_parity(r.distances[sub], r.ids[sub], Dr, Ir, 0, rtol=0.0, atol=0.0,
                      xb=xb, xq=xq[sub])


def test_set_option_rejects_unknown_and_out_of_range(vs):
    """vs_index_set_option takes the documented names only, each within its
    range; a rejected call leaves the index's plan unchanged."""
    idx = vs.GpuIndexFlat.l2(8)
    idx.add(syn.int_grid(100, 8, 1, 0))
    # VS_ERR_INVALID surfaces as ValueError (the reference's ArgumentError)
    with pytest.raises(ValueError, match="unknown option"):
        idx.set_option("no_such_option", 1)
    for name, value in (("gemm", 2), ("km16_rt", 3), ("scan_kkw", -1), ("merge_mu", 3),
                        ("merge_mu", 16), ("prepass_log2", 9), ("prepass_log2", 21),
                        ("merge_g", -1), ("merge_g", 65), ("guess_div_log2", 11)):
        with pytest.raises(ValueError, match="outside"):
            idx.set_option(name, value)
    idx.set_option("guess", 0)
    r = idx.search(syn.int_grid(3, 8, 1, 1), 5)
    idx.close()
    assert r.ids.shape == (3, 5)
