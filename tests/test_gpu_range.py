"""GPU range search and self-join parity against the oracle (restating
IndexFlat.rangeSearch, index_flat.dart:99-137, and the dedup pair list of
bin/vector_dedup_demo.dart:115-128).  Both sides test the fp64 score, so the
CSR results must be identical, distances bit for bit."""
import numpy as np
import pytest

import oracle
from _parity import assert_range_parity
from test_gpu_search import blobs
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def test_range_matches_filtered_knn(vs):
    """vector_store_test.dart:307-329: radius between the 3rd and 4th shell."""
    xb, xq = blobs(400, 16, seed=1), blobs(20, 16, seed=2)
    Dr, _ = oracle.flat_search(xb, xq, 400, 0, NT)
    radius = float((np.float64(Dr[0, 2]) + np.float64(Dr[0, 3])) / 2)
    g = vs.GpuIndexFlat.l2(16)
    g.add(xb)
    rr = g.range_search(xq, radius)
    lims, D, I = oracle.flat_range_search(xb, xq, radius, 0, NT)
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)
    for q in range(20):
        exp = {int(i) for i in np.nonzero((((xq[q].astype(np.float64) - xb) ** 2).sum(1)) <= radius)[0]}
        assert set(rr.ids[rr.limits[q]:rr.limits[q + 1]].tolist()) == exp


@pytest.mark.parametrize("metric,rank", [(0, 3), (0, 60), (1, 5), (1, 200)])
def test_range_parity(vs, metric, rank):
    """radius = the oracle's rank-th score of query 0, so hits exist and one
    query sits exactly on its boundary."""
    xb = blobs(5000, 24, seed=3)
    xq = np.concatenate([xb[:25] + 0.01, blobs(25, 24, seed=4)]).astype(np.float32)
    Dk, _ = oracle.flat_search(xb, xq[:1], rank, metric, 1)
    radius = float(Dk[0, -1])
    g = vs.GpuIndexFlat(24, vs.Metric(metric))
    g.add(xb)
    rr = g.range_search(xq, radius)
    lims, D, I = oracle.flat_range_search(xb, xq, radius, metric, NT)
    assert rr.total_matches > 0
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)


def test_range_at_observed_scores(vs):
    """Radius equal to a stored score: the inclusive fp64 test keeps it."""
    xb = syn.normal_unit(3000, 64, 8, 0)
    xq = syn.normal_unit(10, 64, 8, 1)
    g = vs.GpuIndexFlat.ip(64)
    g.add(xb)
    s = xq[0].astype(np.float64) @ xb[123].astype(np.float64)
    rr = g.range_search(xq, float(s))
    lims, D, I = oracle.flat_range_search(xb, xq, float(s), 1, NT)
    assert 123 in rr.ids[rr.limits[0]:rr.limits[1]].tolist()
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)


def test_range_empty_and_bf16(vs):
    xb16 = syn.to_bf16_bits(syn.normal_unit(20_000, 128, 2, 0))
    xq16 = syn.to_bf16_bits(syn.normal_unit(30, 128, 2, 1))
    g = vs.GpuIndexFlat.ip(128, storage="bf16")
    g.add(xb16)
    rr = g.range_search(xq16, 0.35)
    lims, D, I = oracle.flat_range_search(syn.bf16_bits_to_f32(xb16), syn.bf16_bits_to_f32(xq16), 0.35, 1, NT)
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)
    rr = g.range_search(xq16, 2.0)
    assert rr.total_matches == 0 and rr.nq == 30


@pytest.mark.parametrize("copy16,gemm4", [(1, 0), (0, 0), (1, 1)])
def test_self_join_dedup(vs, opts, copy16, gemm4):
    """configs[4] arithmetic on 30k x 512: 5 % planted near-duplicates,
    pairs i<j with cos >= 0.95, sorted by (i, j).  The one-pass selection
    reads a bf16 copy of the fp32 rows (copy16 1, the default) or rounds
    the fp32 rows in the kernel (0); on the copy, the eight-wave or the
    four-wave GEMM-tiled kernel (gemm4)."""
    opts(copy16=copy16, gemm4=gemm4)
    x = syn.dedup_set(30_000, 512, 0.05, 0.01, 1234)
    g = vs.GpuIndexFlat.ip(512, storage="f32")
    g.add(x)
    i, j, s = g.self_join(0.95)
    ri, rj, rs = oracle.self_join(x, 0.95, nthreads=NT)
    assert len(ri) > 1000
    assert np.array_equal(i, ri) and np.array_equal(j, rj)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("copy16", [1, 0])
def test_range_l2_one_pass_rows(vs, opts, copy16):
    """L2 range search of 600 queries over 20k x 256 fp32 rows on the
    GEMM-tiled one-pass selection (row norms from the fp32 rows), radius at
    the 40th score of query 0: the oracle's CSR result."""
    opts(copy16=copy16)
    xb = blobs(20_000, 256, seed=11)
    xq = np.concatenate([xb[:300] + 0.02, blobs(300, 256, seed=12)]).astype(np.float32)
    Dk, _ = oracle.flat_search(xb, xq[:1], 40, 0, 1)
    radius = float(Dk[0, -1])
    g = vs.GpuIndexFlat.l2(256, storage="f32")
    g.add(xb)
    rr = g.range_search(xq, radius)
    # the GEMM-tiled scan ran on the copy (storage 1) or the fp32 rows (2)
    # (on the copy: the four-wave kernel, or the eight-wave one with it off)
    keys = (["gemm:1,1,2,4,4,2,64", "gemm:1,1,2,2,4,4,32"] if copy16 == 1
            else ["gemm:2,1,2,4,4,2,32"])
    n = sum(g.prof_get(key)[0] for key in keys)
    assert n >= 1
    lims, D, I = oracle.flat_range_search(xb, xq, radius, 0, NT)
    assert rr.total_matches > 0
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)
