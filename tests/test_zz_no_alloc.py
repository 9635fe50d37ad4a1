"""The allocation-free search entry point (vs_index_search_device_noalloc),
called through the C ABI, against the existing vs_index_search_device on the
same index and device buffers: two calls in a row, the second with a smaller
input, each to the parity bar (distances bit-identical, ids equal except in
exact ties), and against the oracle (IndexFlat.search, index_flat.dart:62-97).

Every allocation-free call runs with the test-support countdown "fail_alloc"
armed at 1, so that any device or pinned host allocation the library makes
during the call fails it with VS_ERR_OOM.
"""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity
from vector_store import _native as NN
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def _search(idx, entry, q, k, dtype):
    nq = q.shape[0]
    qb, Db, Ib = NN.DeviceBuffer(q.nbytes), NN.DeviceBuffer(nq * k * 4), NN.DeviceBuffer(nq * k * 4)
    armed = entry.endswith("_noalloc")
    try:
        qb.upload(q)
        if armed:  # the next allocation of this thread fails the call
            idx.set_option("fail_alloc", 1)
        try:
            NN.check(getattr(NN.load(), entry)(idx.handle, qb.ptr, dtype, nq, k, Db.ptr, Ib.ptr))
        finally:
            if armed:
                idx.set_option("fail_alloc", 0)
        D = np.empty((nq, k), np.float32)
        I = np.empty((nq, k), np.int32)
        Db.download(D)
        Ib.download(I)
    finally:
        for b in (qb, Db, Ib):
            b.free()
    return D, I


def _check(idx, q, k, metric, dtype, xb32, q32, rtol):
    D0, I0 = _search(idx, "vs_index_search_device", q, k, dtype)
    D1, I1 = _search(idx, "vs_index_search_device_noalloc", q, k, dtype)
    assert_knn_parity(D1, I1, D0, I0, metric, rtol=0.0, atol=0.0)
    Dr, Ir = oracle.flat_search(xb32, q32, k, metric, NT)
    assert_knn_parity(D1, I1, Dr, Ir, metric, rtol=rtol)


def test_noalloc_matches_search_device_bf16_ip():
    """bf16 unit rows (configs[2] arithmetic), 300k x 768, IP: batch 64 with
    k = 100 (threshold seeding runs), then batch 7 with k = 10."""
    xb16 = syn.to_bf16_bits(syn.normal_unit(300_000, 768, 31, 0))
    xq16 = syn.to_bf16_bits(syn.normal_unit(64, 768, 31, 1))
    import vector_store as vs

    idx = vs.GpuIndexFlat(768, vs.Metric.innerProduct, storage="bf16")
    try:
        idx.add(xb16)
        xb32 = syn.bf16_bits_to_f32(xb16)
        _check(idx, xq16, 100, 1, NN.VS_DTYPE_BF16, xb32, syn.bf16_bits_to_f32(xq16), 1e-3)
        _check(idx, xq16[:7], 10, 1, NN.VS_DTYPE_BF16, xb32, syn.bf16_bits_to_f32(xq16[:7]), 1e-3)
    finally:
        idx.close()


def test_noalloc_exact_fallback_fp32_l2():
    """fp32 rows with near-duplicates of the queries (every query takes the
    exact path): 12 queries, k = 10, then 3 queries, k = 5."""
    import vector_store as vs

    g = syn.rng(5, 11)
    q = g.standard_normal((12, 256)).astype(np.float32)
    cop = np.repeat(q, 32, axis=0) + g.standard_normal((12 * 32, 256)).astype(np.float32) * 1e-4
    xb = np.concatenate([g.standard_normal((30_000, 256)).astype(np.float32), cop])
    idx = vs.GpuIndexFlat(256, vs.Metric.l2, storage="f32")
    try:
        idx.add(xb)
        _check(idx, q, 10, 0, NN.VS_DTYPE_F32, xb, q, 0.0)
        _check(idx, q[:3], 5, 0, NN.VS_DTYPE_F32, xb, q[:3], 0.0)
    finally:
        idx.close()


def test_noalloc_limits():
    import vector_store as vs

    idx = vs.GpuIndexFlat(16, vs.Metric.l2, storage="f32")
    try:
        idx.add(np.ones((10, 16), np.float32))
        q = np.ones((65, 16), np.float32)
        with pytest.raises(NotImplementedError):
            _search(idx, "vs_index_search_device_noalloc", q, 4, NN.VS_DTYPE_F32)
        with pytest.raises(NotImplementedError):
            _search(idx, "vs_index_search_device_noalloc", q[:2], 129, NN.VS_DTYPE_F32)
        D, I = _search(idx, "vs_index_search_device_noalloc", q[:2], 12, NN.VS_DTYPE_F32)
        assert np.all(I[:, 10:] == -1) and np.all(D[:, :10] == 0.0)
    finally:
        idx.close()
