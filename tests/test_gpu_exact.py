"""Exactness of the top-k selection where the MFMA accumulator cannot decide,
and top-k for any k (TopK, lib/core/vector_store/index.dart:213-331, accepts
every k; vector_store_test.dart:307-329 searches with k = ntotal).

The fused search selects candidates by the MFMA accumulator and re-ranks them
in fp64.  Its merge proves, per query, that no row it dropped could beat the
k-th exact result (the accumulator's error bound against the gap to the
kk-th kept value); queries it cannot prove go to an exact path that scores
every row in the reference's fp64 arithmetic.  Large k sorts every row's
exact key."""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def near_copies(nbase, ncopy, nrand, d, sigma, seed):
    """Queries, each with ncopy copies plus N(0, sigma^2) noise in the
    database, among nrand unrelated N(0,1) rows (fp32, not normalised)."""
    g = syn.rng(seed, 11)
    q = g.standard_normal((nbase, d)).astype(np.float32)
    cop = (np.repeat(q, ncopy, axis=0) +
           g.standard_normal((nbase * ncopy, d)).astype(np.float32) * np.float32(sigma))
    rnd = g.standard_normal((nrand, d)).astype(np.float32)
    xb = np.concatenate([rnd[: nrand // 2], cop, rnd[nrand // 2:]]).astype(np.float32)
    return xb, q


@pytest.mark.parametrize("metric", [0, 1])
def test_near_duplicates_go_exact(vs, metric):
    """fp32 rows, d = 768, 64 copies of each query with N(0, 1e-4^2) noise:
    neighbours closer together than the accumulator's error.  Results equal
    the oracle's (no tolerance: distances bit-exact, ids per exact tie)."""
    xb, xq = near_copies(12, 64, 20_000, 768, 1e-4, 5)
    idx = vs.GpuIndexFlat(768, vs.Metric(metric), storage="f32")
    idx.add(xb)
    idx.prof_reset()
    r = idx.search(xq, 10)
    nx = idx.prof_get("exact_fallback")[0]
    idx.close()
    Dr, Ir = oracle.flat_search(xb, xq, 10, metric, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, metric, rtol=0.0, atol=0.0)
    if metric == 0:
        # the L2 gaps (~1e-6 on distances ~1.5e-5) are far inside the bound
        assert nx == len(xq), f"{nx} of {len(xq)} queries took the exact path"


def test_exact_path_bf16_two_planes(vs):
    """bf16 rows, fp32 queries (two query planes) near stored rows: the
    exact path reads bf16 rows."""
    xb, xq = near_copies(8, 32, 50_000, 256, 1e-3, 9)
    xb16 = syn.to_bf16_bits(xb)
    idx = vs.GpuIndexFlat(256, vs.Metric.l2, storage="bf16")
    idx.add(xb16)
    r = idx.search(xq, 16)
    idx.close()
    Dr, Ir = oracle.flat_search(syn.bf16_bits_to_f32(xb16), xq, 16, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0, rtol=0.0, atol=0.0)


@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("k", [1000, 3000, 3500])
def test_large_k(vs, metric, k):
    """k = 1000, k = ntotal and k > ntotal (sentinels) on 3000 x 32 rows."""
    g = syn.rng(21, 0)
    xb = g.standard_normal((3000, 32)).astype(np.float32)
    xq = g.standard_normal((7, 32)).astype(np.float32)
    idx = vs.GpuIndexFlat(32, vs.Metric(metric), storage="f32")
    idx.add(xb)
    r = idx.search(xq, k)
    idx.close()
    Dr, Ir = oracle.flat_search(xb, xq, k, metric, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, metric, rtol=0.0, atol=0.0)


def test_large_k_device_buffers(vs):
    """k = 600 through the device-buffer entry point, bf16 storage, IP."""
    from vector_store import _native as NN

    xb16 = syn.to_bf16_bits(syn.normal_unit(20_000, 128, 3, 0))
    xq16 = syn.to_bf16_bits(syn.normal_unit(5, 128, 3, 1))
    idx = vs.GpuIndexFlat(128, vs.Metric.innerProduct, storage="bf16")
    idx.add(xb16)
    k = 600
    qb, Db, Ib = NN.DeviceBuffer(xq16.nbytes), NN.DeviceBuffer(5 * k * 4), NN.DeviceBuffer(5 * k * 4)
    qb.upload(xq16)
    idx.search_device(qb, 5, k, Db, Ib, NN.VS_DTYPE_BF16)
    D = np.empty((5, k), np.float32)
    I = np.empty((5, k), np.int32)
    Db.download(D)
    Ib.download(I)
    for b in (qb, Db, Ib):
        b.free()
    idx.close()
    Dr, Ir = oracle.flat_search(syn.bf16_bits_to_f32(xb16), syn.bf16_bits_to_f32(xq16), k, 1, NT)
    assert_knn_parity(D, I, Dr, Ir, 1, rtol=0.0, atol=0.0)


def test_bound_check_passes_on_spread_data(vs):
    """Unrelated rows: the proof succeeds and no query needs the exact path."""
    xb = syn.int_grid(200_000, 128, 4, 0)
    xq = syn.int_grid(300, 128, 4, 1)
    idx = vs.GpuIndexFlat.l2(128)
    idx.add(xb)
    idx.prof_reset()
    r = idx.search(xq, 100)
    nx = idx.prof_get("exact_fallback")[0]
    idx.close()
    Dr, Ir = oracle.flat_search(xb, xq, 100, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0)
    assert nx == 0
