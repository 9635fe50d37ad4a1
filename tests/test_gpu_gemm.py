"""Parity of the GEMM-tiled distance scan (large query batches, both operands
staged in LDS) against the CPU oracle (restating IndexFlat.search /
rangeSearch, index_flat.dart:62-137, and the Kmeans assign/update steps,
kmeans.dart:91-140).

Every built shape is forced here: bf16 rows with one or two query planes
(K-chunks of 64 in XOR-swizzled LDS rows, or 32 in padded ones),
fp32 rows (split into bf16 hi/lo planes in LDS) with one or two query
planes, 128- and 256-query blocks, 4 and 8 waves.  Row counts end inside a
row tile, query counts inside a query block, d is ragged, both metrics, k
from 1 to 100.  Each test also checks, through the always-on "gemm" launch
counters, that the GEMM-tiled kernel really ran in the forced shape."""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity, assert_range_parity
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()

# The built shapes (storage, query planes, row waves, query waves, 32-row
# blocks per wave, 32-query blocks per wave, K-chunk), as listed by
# VS_GEMM_SHAPES in dart-pytorch_amd/csrc/vs_internal.h, and first the
# four-wave pipelined kernel (bf16 rows, one query plane; option gemm4).
SHAPES = [
    (1, 1, 2, 2, 4, 4, 32),  # the four-wave pipelined kernel
    (1, 1, 2, 4, 4, 2, 64),
    (1, 1, 2, 2, 4, 2, 64),
    (1, 1, 2, 4, 4, 2, 32),
    (1, 1, 2, 2, 4, 2, 32),
    (1, 2, 2, 4, 4, 2, 32),
    (1, 2, 2, 2, 4, 2, 32),
    (0, 2, 2, 4, 4, 2, 16),
    (0, 2, 2, 2, 4, 2, 32),
    (0, 1, 2, 4, 4, 2, 32),
    (0, 1, 2, 2, 4, 2, 32),
]


def _key(shape):
    return "gemm:" + ",".join(map(str, shape))


@pytest.fixture(autouse=True)
def _gemm(opts):
    """The GEMM-tiled scan is switched on for every test here (the row-shared
    scan, planned before it, off)."""
    opts(gemm=1, share=0, gemm_min_nq=256)


def _force(opts, shape):
    """Force one GEMM shape (32-query blocks per wave = 4: the four-wave
    kernel, option gemm4)."""
    _, _, _, wq, _, qb, kc = shape
    opts(gemm_wq=wq, gemm_qb=qb, gemm_kc=kc, gemm4=int(qb == 4))


def _search(vs, xb, xq, k, metric, storage, shape=None, key=None):
    idx = vs.GpuIndexFlat(xb.shape[1], vs.Metric(metric), storage=storage)
    idx.add(xb)
    r = idx.search(xq, k)
    gemm, _ = idx.prof_get("gemm")
    if shape is not None or key is not None:
        key = key or _key(shape)
        n, _ = idx.prof_get(key)
        assert n >= 1, f"{key} did not run"
    idx.close()
    return r.distances, r.ids, gemm


def _inputs(shape, d, seed, n=9000, nq=300):
    """Rows and queries whose storage and query planes select `shape`: bf16
    rows (bf16 bits) or fp32 rows; bf16-exact or general fp32 queries.
    9,000 rows end inside a row tile and 300 queries inside a query block."""
    st, pb = shape[0], shape[1]
    xb = syn.normal_unit(n, d, seed, 0)
    xq = syn.normal_unit(nq, d, seed, 1)
    if st == 1:
        xb = syn.to_bf16_bits(xb)
    if pb == 1:
        xq = syn.bf16_bits_to_f32(syn.to_bf16_bits(xq))
    return xb, xq, ("bf16" if st == 1 else "f32")


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "-".join(map(str, s)))
@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("k,d", [(10, 200), (100, 768), (1, 72)])
def test_gemm_shape_parity(vs, opts, shape, metric, k, d):
    _force(opts, shape)
    xb, xq, storage = _inputs(shape, d, 31 + metric)
    D, I, gemm = _search(vs, xb, xq, k, metric, storage, shape)
    assert gemm >= 1
    xbf = syn.bf16_bits_to_f32(xb) if storage == "bf16" else xb
    Dr, Ir = oracle.flat_search(xbf, xq, k, metric, NT)
    assert_knn_parity(D, I, Dr, Ir, metric, rtol=1e-3 if storage == "bf16" else 1e-5)


@pytest.mark.parametrize("kc", [64, 32])
@pytest.mark.parametrize("wq,qb", [(4, 2), (2, 2)])
def test_gemm_config2_exact(vs, opts, wq, qb, kc):
    """configs[1] arithmetic on a 100k slice with 1,000 queries: integer
    distances, bit-exact, k = 100, with K-chunks of 64 and 32."""
    opts(gemm_wq=wq, gemm_qb=qb, gemm_kc=kc)
    xb = syn.int_grid(100_000, 128, 1234, 0)
    xq = syn.int_grid(1000, 128, 1234, 1)
    key = _key((1, 1, 2, wq, 4, qb, kc))
    D, I, gemm = _search(vs, xb, xq, 100, 0, "auto", key=key)
    assert gemm >= 1
    Dr, Ir = oracle.flat_search(xb, xq, 100, 0, NT)
    assert_knn_parity(D, I, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)
    assert np.all(D == np.round(D))


def test_gemm_matches_streaming(vs, opts):
    """Same inputs through the GEMM-tiled and streaming scans give the same
    answers (integer data: exact distances)."""
    xb = syn.int_grid(30_000, 64, 3, 0)
    xq = syn.int_grid(700, 64, 3, 1)
    D1, I1, g1 = _search(vs, xb, xq, 16, 0, "auto")
    opts(gemm=0)
    D0, I0, g0 = _search(vs, xb, xq, 16, 0, "auto")
    assert g1 >= 1 and g0 == 0
    assert np.array_equal(D0, D1)
    Dr, Ir = oracle.flat_search(xb, xq, 16, 0, NT)
    assert_knn_parity(D1, I1, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)


@pytest.mark.parametrize("metric", [0, 1])
def test_four_wave_matches_eight_wave(vs, opts, metric):
    """The four-wave pipelined kernel (option gemm4) and the eight-wave one
    give the same answers on bf16 rows of integers (exact distances), k =
    100, 50,001 rows (ending inside a 256-row tile) and 777 queries (inside
    a 256-query block), both equal to the oracle's."""
    xb = syn.int_grid(50_001, 128, 5, 0)
    xq = syn.int_grid(777, 128, 5, 1)
    opts(gemm_min_nq=256)
    D8, I8, g8 = _search(vs, xb, xq, 100, metric, "auto", key="gemm:1,1,2,4,4,2,64")
    opts(gemm4=1)
    D4, I4, g4 = _search(vs, xb, xq, 100, metric, "auto", key="gemm:1,1,2,2,4,4,32")
    assert np.array_equal(D8, D4) and np.array_equal(I8, I4)
    Dr, Ir = oracle.flat_search(xb, xq, 100, metric, NT)
    assert_knn_parity(D4, I4, Dr, Ir, metric, rtol=0.0, atol=0.0, xb=xb, xq=xq)


@pytest.mark.parametrize("k,metric", [(10, 0), (100, 1)])
def test_gemm_estimated_threshold_sample(vs, opts, k, metric):
    """A large batch over 2^18+ rows on the GEMM-tiled scan starts from a
    threshold estimated on the first 1/2^g of the rows (option
    guess_div_log2; 1/32 by default): every sample size gives
    the oracle's result, with one estimate pre-pass and no exact re-search.
    A sample of 2^16 rows or more (here 1/2) is itself seeded by a bound from
    its first 1/32 (one more pre-pass scan)."""
    xb = syn.int_grid(300_000, 64, 17, 0)
    xq = syn.int_grid(600, 64, 17, 1)
    res = {}
    for g in (0, 1, 5, 7, 10):
        opts(guess_div_log2=g)
        idx = vs.GpuIndexFlat(64, vs.Metric(metric), storage="auto")
        idx.add(xb)
        idx.prof_enable(True)
        r = idx.search(xq, k)
        ng, _ = idx.prof_get("guess_scans")
        npre, _ = idx.prof_get("prepass_scans")
        nfb, _ = idx.prof_get("fallback")
        ngm, _ = idx.prof_get("gemm")
        idx.close()
        assert ng == 1 and nfb == 0 and ngm >= 1, (g, ng, nfb, ngm)
        assert npre == (2 if g == 1 else 1), (g, npre)
        res[g] = r
    sub = np.arange(0, 600, 5)
    Dr, Ir = oracle.flat_search(xb, xq[sub], k, metric, NT)
    for g, r in res.items():
        assert_knn_parity(r.distances[sub], r.ids[sub], Dr, Ir, metric, rtol=0.0, atol=0.0,
                          xb=xb, xq=xq[sub])
        assert np.array_equal(r.distances, res[5].distances), g


def test_gemm_verification_path(vs, opts):
    """Lists forced down to 4 entries (option scan_kkw) with k = 60: the merge
    must detect queries whose lists may have dropped a winner and search
    them again; the answer stays exact."""
    opts(scan_kkw=4)
    xb = syn.int_grid(20_000, 64, 5, 0)
    xq = syn.int_grid(300, 64, 5, 1)
    D, I, gemm = _search(vs, xb, xq, 60, 0, "auto")
    assert gemm >= 1
    Dr, Ir = oracle.flat_search(xb, xq, 60, 0, NT)
    assert_knn_parity(D, I, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)


def test_gemm_query_blocks_past_padding(vs):
    """1,300 queries in 256-query blocks: the last block reaches query row
    1,535, inside the prepared-query padding."""
    xb16 = syn.to_bf16_bits(syn.normal_unit(5000, 768, 41, 0))
    xq16 = syn.to_bf16_bits(syn.normal_unit(1300, 768, 41, 1))
    D, I, gemm = _search(vs, xb16, xq16, 10, 1, "bf16")
    assert gemm >= 1
    Dr, Ir = oracle.flat_search(syn.bf16_bits_to_f32(xb16), syn.bf16_bits_to_f32(xq16), 10, 1, NT)
    assert_knn_parity(D, I, Dr, Ir, 1, rtol=1e-3)


@pytest.mark.parametrize("metric", [0, 1])
def test_gemm_range_search(vs, metric):
    """Range search with 600 queries runs on the GEMM-tiled kernel (MODE 1)."""
    xb = syn.normal_unit(8000, 96, 17, 0)
    xq = np.concatenate([xb[:300] + 0.02, syn.normal_unit(300, 96, 17, 1)]).astype(np.float32)
    radius = 0.05 if metric == 0 else 0.6
    g = vs.GpuIndexFlat(96, vs.Metric(metric), storage="f32")
    g.add(xb)
    rr = g.range_search(xq, radius)
    gemm, _ = g.prof_get("gemm")
    g.close()
    assert gemm >= 1
    lims, D, I = oracle.flat_range_search(xb, xq, radius, metric, NT)
    assert lims[-1] >= 300
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)


def test_gemm_self_join(vs):
    """Self-join (upper triangle, MODE 1) of 3,000 unit vectors with planted
    near-duplicates on the GEMM-tiled kernel: the pair list equals the
    oracle's range search filtered to i < j."""
    base = syn.normal_unit(2800, 64, 23, 0)
    rng = np.random.default_rng(23)
    src = rng.integers(0, 2800, 200)
    dup = base[src] + rng.normal(0, 0.01, (200, 64)).astype(np.float32)
    dup /= np.linalg.norm(dup.astype(np.float64), axis=1, keepdims=True).astype(np.float32)
    xb = np.concatenate([base, dup.astype(np.float32)])
    g = vs.GpuIndexFlat(64, vs.Metric(1), storage="f32")
    g.add(xb)
    i, j, s = g.self_join(0.95)
    gemm, _ = g.prof_get("gemm")
    g.close()
    assert gemm >= 1
    ri, rj, rs = oracle.self_join(xb, 0.95, nthreads=NT)
    assert len(ri) >= 200
    assert np.array_equal(i, ri) and np.array_equal(j, rj)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_gemm_kmeans_step(vs):
    """k-means steps with 20,000 points as queries run on the GEMM-tiled
    kernel (fp32 rows, two query planes): assignments, objective and
    centroids bit-identical to the oracle's."""
    x, _ = syn.gaussian_mixture(20_000, 256, 64, 0.1, 1234)
    cen = x[syn.seeded_subset(len(x), 256, 1234)].copy()
    pts = vs.GpuIndexFlat.l2(256, storage="f32")
    pts.add(x)
    for it in range(2):
        u = syn.rng(77, it).random(256 * 256)
        a, newc, cnt, obj = vs.kmeans_step(pts, cen, 1, u)
        ar, _, objr = oracle.kmeans_assign(x, cen, NT)
        assert np.array_equal(a, ar), f"iteration {it}: {np.sum(a != ar)} assignments differ"
        assert obj == objr
        cr, cntr, _ = oracle.kmeans_update(x, ar, cen, 1, u)
        assert np.array_equal(cnt, cntr)
        assert np.array_equal(newc.view(np.uint32), cr.view(np.uint32))
        cen = newc
    gemm, _ = pts.prof_get("gemm")
    pts.close()
    assert gemm >= 2


def test_gemm_large_k_unseeded(vs):
    """k = 300: lists keep 256 entries, more than the two lanes of a list
    hold in one tile, so the first tile is not seeded (the plain append
    path runs from the start); the answer stays exact."""
    xb = syn.int_grid(40_000, 64, 9, 0)
    xq = syn.int_grid(300, 64, 9, 1)
    D, I, gemm = _search(vs, xb, xq, 300, 0, "auto")
    assert gemm >= 1
    Dr, Ir = oracle.flat_search(xb, xq, 300, 0, NT)
    assert_knn_parity(D, I, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)


# one-pass selection shapes: fp32 rows rounded in the kernel (storage code 2)
# or their bf16 copy (storage code 1, range search and self-join)
COARSE_KEYS = ("gemm:2,1,2,4,4,2,32", "gemm:1,1,2,4,4,2,64", "gemm:1,1,2,4,4,2,32",
               "gemm:1,1,2,2,4,4,32")


def _one_pass_runs(g):
    return sum(g.prof_get(k)[0] for k in COARSE_KEYS)


@pytest.mark.parametrize("coarse", [1, 0])
def test_coarse_self_join(vs, opts, coarse):
    """configs[4] shape at 4,000 rows (d = 512, 5% planted copies, cos >=
    0.95): the one-pass selection (bf16 hi planes, widened margins, exact
    fp64 re-test) and the three-pass one give the oracle's pair list."""
    opts(gemm=-1, coarse=coarse)  # the default planner rule
    x = syn.dedup_set(4000, 512, 0.05, 0.01, 11)
    g = vs.GpuIndexFlat(512, vs.Metric(1), storage="f32")
    g.add(x)
    i, j, s = g.self_join(0.95)
    n1 = _one_pass_runs(g)
    gemm, _ = g.prof_get("gemm")
    g.close()
    assert gemm >= 1 and (n1 >= 1) == bool(coarse)
    ri, rj, rs = oracle.self_join(x, 0.95, nthreads=NT)
    assert len(ri) >= 200
    assert np.array_equal(i, ri) and np.array_equal(j, rj)
    assert np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("coarse", [1, 0])
def test_coarse_kmeans(vs, opts, coarse):
    """configs[3] arithmetic at 30,000 points (d = 256, 1,024 mixture
    components, 4,096 centroids): assignments, objective and centroids equal
    the oracle's with and without the one-pass selection."""
    opts(gemm=-1, coarse=coarse)
    x, _ = syn.gaussian_mixture(30_000, 256, 1024, 0.1, 77)
    cen = x[syn.seeded_subset(len(x), 4096, 77)].copy()
    pts = vs.GpuIndexFlat.l2(256, storage="f32")
    pts.add(x)
    u = syn.rng(78, 0).random(4096 * 256)
    a, newc, cnt, obj = vs.kmeans_step(pts, cen, 1, u)
    n1 = _one_pass_runs(pts)
    pts.close()
    assert (n1 >= 1) == bool(coarse)
    ar, _, objr = oracle.kmeans_assign(x, cen, NT)
    assert np.array_equal(a, ar), f"{np.sum(a != ar)} assignments differ"
    assert obj == objr
    cr, cntr, _ = oracle.kmeans_update(x, ar, cen, 1, u)
    assert np.array_equal(cnt, cntr)
    assert np.array_equal(newc.view(np.uint32), cr.view(np.uint32))


@pytest.mark.parametrize("metric", [0, 1])
def test_coarse_range_search(vs, opts, metric):
    """Range search of 700 fp32 queries (d = 256) on the one-pass selection:
    the CSR result equals the oracle's bit for bit."""
    opts(gemm=-1)
    xb = syn.normal_unit(6000, 256, 19, 0)
    xq = np.concatenate([xb[:350] + 0.01, syn.normal_unit(350, 256, 19, 1)]).astype(np.float32)
    radius = 0.05 if metric == 0 else 0.5
    g = vs.GpuIndexFlat(256, vs.Metric(metric), storage="f32")
    g.add(xb)
    rr = g.range_search(xq, radius)
    n1 = _one_pass_runs(g)
    g.close()
    assert n1 >= 1
    lims, D, I = oracle.flat_range_search(xb, xq, radius, metric, NT)
    assert lims[-1] >= 350
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)


@pytest.mark.parametrize("coarse", [1, 0])
def test_kmeans_exhaustive_fallback(vs, opts, coarse):
    """Twenty identical copies of one centroid fill the 16-entry shortlist
    of the points near it, so their pick cannot be proven and the exhaustive
    exact scan runs: the answer is the lowest index among the copies (the
    strict '<' scan, kmeans.dart:93-101), as the oracle gives."""
    opts(gemm=-1, coarse=coarse)
    x, _ = syn.gaussian_mixture(6000, 256, 16, 0.1, 5)
    cen = x[syn.seeded_subset(len(x), 300, 5)].copy()
    cen[100:120] = cen[3]  # 20 copies of centroid 3
    pts = vs.GpuIndexFlat.l2(256, storage="f32")
    pts.add(x)
    a, newc, cnt, obj = vs.kmeans_step(pts, cen, 1, syn.rng(6, 0).random(300 * 256))
    nfb, _ = pts.prof_get("kmeans_fallback_points")
    pts.close()
    assert nfb >= 1
    ar, _, objr = oracle.kmeans_assign(x, cen, NT)
    assert np.array_equal(a, ar) and obj == objr
    assert not np.any((a >= 100) & (a < 120))  # copies lose to centroid 3

