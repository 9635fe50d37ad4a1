"""Failure paths of the C ABI on the GPU: oversize requests and device
allocation failures (forced through the test-support option "fail_alloc",
which makes the n-th allocation of this thread report out-of-memory).

Every failed call must return its status without side effects -- an add
that fails stores nothing -- and the same index must then give the oracle's
results (index_flat.dart:62-137 for search and range search, kmeans.dart:91-140
for the k-means step)."""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity, assert_range_parity
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def _oom(vs, fn):
    with pytest.raises(vs.VsError) as e:
        fn()
    assert e.value.code == vs._native.VS_ERR_OOM, str(e.value)


def test_oversize_reserve(vs):
    """More rows than int32 ids can name is invalid; a representable but
    impossible reservation (2^31 - 1 rows of 16 KiB) is out of memory; the
    index stays usable."""
    idx = vs.GpuIndexFlat.l2(4096, storage="f32")
    with pytest.raises(ValueError, match="int32"):
        idx.reserve(1 << 31)
    _oom(vs, lambda: idx.reserve((1 << 31) - 1))
    xb = syn.int_grid(300, 4096, 1, 0)
    xq = syn.int_grid(4, 4096, 1, 1)
    idx.add(xb)
    r = idx.search(xq, 5)
    idx.close()
    Dr, Ir = oracle.flat_search(xb, xq, 5, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)


def test_add_allocation_failure_stores_nothing(vs):
    xb = syn.int_grid(2000, 64, 2, 0)
    idx = vs.GpuIndexFlat.l2(64)
    idx.set_option("fail_alloc", 1)
    _oom(vs, lambda: idx.add(xb))
    idx.set_option("fail_alloc", 0)
    assert idx.ntotal == 0
    idx.add(xb)
    assert idx.ntotal == 2000
    xq = syn.int_grid(7, 64, 2, 1)
    r = idx.search(xq, 10)
    idx.close()
    Dr, Ir = oracle.flat_search(xb, xq, 10, 0, NT)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)


@pytest.mark.parametrize("nq", [5, 600])
def test_search_allocation_failures(vs, nq):
    """The first search of an index allocates its scratch; the n-th of those
    allocations fails for n = 1, 2, ...: each failed search reports
    out-of-memory, and the next one, with nothing forced, is exact."""
    xb = syn.int_grid(5000, 128, 3, 0)
    xq = syn.int_grid(nq, 128, 3, 1)
    Dr, Ir = oracle.flat_search(xb, xq, 20, 0, NT)
    failed = 0
    for n in range(1, 12):
        idx = vs.GpuIndexFlat.l2(128)
        idx.add(xb)
        idx.set_option("fail_alloc", n)
        try:
            idx.search(xq, 20)
        except vs.VsError as e:
            assert e.code == vs._native.VS_ERR_OOM
            failed += 1
        idx.set_option("fail_alloc", 0)
        r = idx.search(xq, 20)
        idx.close()
        assert_knn_parity(r.distances, r.ids, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)
    assert failed >= 1


def test_range_and_kmeans_allocation_failures(vs):
    xb = syn.normal_unit(3000, 64, 4, 0)
    xq = np.concatenate([xb[:20] + 0.01, syn.normal_unit(20, 64, 4, 1)]).astype(np.float32)
    lims, D, I = oracle.flat_range_search(xb, xq, 0.05, 0, NT)
    idx = vs.GpuIndexFlat.l2(64, storage="f32")
    idx.add(xb)
    idx.set_option("fail_alloc", 1)
    _oom(vs, lambda: idx.range_search(xq, 0.05))
    idx.set_option("fail_alloc", 0)
    rr = idx.range_search(xq, 0.05)
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)

    cen = xb[:50].copy()
    u = syn.rng(5, 0).random(50 * 64)
    idx.set_option("fail_alloc", 1)
    _oom(vs, lambda: vs.kmeans_step(idx, cen, 1, u))
    idx.set_option("fail_alloc", 0)
    a, newc, cnt, obj = vs.kmeans_step(idx, cen, 1, u)
    idx.close()
    ar, _, objr = oracle.kmeans_assign(xb, cen, NT)
    assert np.array_equal(a, ar) and obj == objr


def test_device_probes(vs):
    """vs_dev_probe: read bandwidth (what 0), bf16 MFMA rate on small-integer
    (1) and random (2) operands, all positive and below the published peaks
    (8 TB/s, 2.5 PFLOP/s); other codes are rejected."""
    import ctypes
    from vector_store import _native as N

    lib = N.load()
    vals = {}
    for what, nbytes in ((0, 1 << 28), (1, 0), (2, 0)):
        v = ctypes.c_double(0.0)
        assert lib.vs_dev_probe(0, what, nbytes, ctypes.byref(v)) == 0
        vals[what] = v.value
    assert 500.0 < vals[0] < 8000.0
    assert 100.0 < vals[1] <= 2600.0 and 100.0 < vals[2] <= 2600.0
    v = ctypes.c_double(0.0)
    assert lib.vs_dev_probe(0, 3, 0, ctypes.byref(v)) == N.VS_ERR_INVALID
