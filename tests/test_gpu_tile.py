"""Parity of the LDS-tiled distance scan (large query batches) against the CPU
oracle (restating IndexFlat.search / rangeSearch, index_flat.dart:62-137).

Every shape the planner can pick is forced here: bf16 rows with one or two
query planes, fp32 rows (split into bf16 hi/lo planes in LDS), 128- and
256-query blocks, 128- and 256-row tiles, row counts that end inside a tile,
ragged d, both metrics, k from 1 to 100.  Each test also checks, through the
always-on "tiled" launch counter, that the tiled kernel really ran."""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity, assert_range_parity
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


# The built shapes (storage, query planes, 32-query blocks, 32-row blocks per
# wave, K-chunk, waves per workgroup), as listed by VS_TILE_SHAPES in
# dart-pytorch_amd/csrc/vs_internal.h.  The block's query planes stay in LDS.
SHAPES = [
    (1, 1, 4, 2, 64, 4),
    (1, 1, 4, 2, 32, 8),
    (1, 1, 3, 2, 64, 4),
    (1, 1, 3, 2, 32, 8),
    (1, 1, 2, 2, 64, 4),
    (1, 2, 2, 2, 64, 4),
    (0, 2, 4, 2, 32, 4),
    (0, 2, 2, 2, 32, 4),
    (0, 1, 4, 2, 32, 4),
    (0, 1, 2, 2, 32, 4),
]


@pytest.fixture(autouse=True)
def _tiled(monkeypatch):
    """The tiled scan is opt-in (VS_TILE=1); every test here turns it on, and
    the GEMM-tiled scan (planned before it for large batches) off."""
    monkeypatch.setenv("VS_TILE", "1")
    monkeypatch.setenv("VS_GEMM", "0")
    monkeypatch.setenv("VS_SHARE", "0")


def _force(monkeypatch, shape):
    st, pb, qb, rb, kc, nw = shape
    for name, v in (("QB", qb), ("RB", rb), ("KC", kc), ("NW", nw)):
        monkeypatch.setenv("VS_TILE_" + name, str(v))


def _search(vs, xb, xq, k, metric, storage, shape=None):
    idx = vs.GpuIndexFlat(xb.shape[1], vs.Metric(metric), storage=storage)
    idx.add(xb)
    r = idx.search(xq, k)
    tiled, _ = idx.prof_get("tiled")
    streamed, _ = idx.prof_get("streamed")
    if shape is not None:
        n, _ = idx.prof_get("tile:" + ",".join(map(str, shape)))
        assert n >= 1, f"shape {shape} did not run"
    idx.close()
    return r.distances, r.ids, tiled, streamed


def _inputs(shape, seed):
    """Rows and queries whose storage and query planes select `shape`:
    bf16 rows (bf16 bits) or fp32 rows; bf16-exact or general fp32 queries.
    d = 768 where the resident query planes fit, else 200 or
    120 (ragged); 9,000 rows end inside a row tile."""
    st, pb, qb, _, _, _ = shape
    planes_bytes = {1: 2, 2: 4}[pb] * 32 * qb
    d = 768 if planes_bytes * 776 <= 150 * 1024 else (200 if planes_bytes * 264 <= 150 * 1024 else 120)
    xb = syn.normal_unit(9000, d, seed, 0)
    xq = syn.normal_unit(300, d, seed, 1)
    if st == 1:
        xb = syn.to_bf16_bits(xb)
    if pb == 1:
        xq = syn.bf16_bits_to_f32(syn.to_bf16_bits(xq))
    return xb, xq, ("bf16" if st == 1 else "f32")


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "-".join(map(str, s)))
@pytest.mark.parametrize("metric", [0, 1])
@pytest.mark.parametrize("k", [10, 100])
def test_tile_shape_parity(vs, monkeypatch, shape, metric, k):
    _force(monkeypatch, shape)
    xb, xq, storage = _inputs(shape, 31 + metric)
    D, I, tiled, _ = _search(vs, xb, xq, k, metric, storage, shape)
    assert tiled >= 1
    xbf = syn.bf16_bits_to_f32(xb) if storage == "bf16" else xb
    Dr, Ir = oracle.flat_search(xbf, xq, k, metric, NT)
    assert_knn_parity(D, I, Dr, Ir, metric, rtol=1e-3 if storage == "bf16" else 1e-5)


@pytest.mark.parametrize("nw", [4, 8])
def test_tile_config2_exact(vs, monkeypatch, nw):
    """configs[1] arithmetic on a 100k slice with 1,000 queries: integer
    distances, bit-exact, k = 100, with 4 or 8 waves per workgroup."""
    monkeypatch.setenv("VS_TILE_NW", str(nw))
    xb = syn.int_grid(100_000, 128, 1234, 0)
    xq = syn.int_grid(1000, 128, 1234, 1)
    D, I, tiled, _ = _search(vs, xb, xq, 100, 0, "auto")
    assert tiled >= 1
    Dr, Ir = oracle.flat_search(xb, xq, 100, 0, NT)
    assert_knn_parity(D, I, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)
    assert np.all(D == np.round(D))


def test_tile_matches_streaming(vs, monkeypatch):
    """Same inputs through both scan kernels give the same answers."""
    xb = syn.int_grid(30_000, 64, 3, 0)
    xq = syn.int_grid(400, 64, 3, 1)
    D1, I1, t1, s1 = _search(vs, xb, xq, 16, 0, "auto")
    monkeypatch.setenv("VS_TILE", "0")
    D0, I0, t0, s0 = _search(vs, xb, xq, 16, 0, "auto")
    assert t1 >= 1 and s0 >= 1 and t0 == 0
    assert np.array_equal(D0, D1)
    Dr, Ir = oracle.flat_search(xb, xq, 16, 0, NT)
    assert_knn_parity(D1, I1, Dr, Ir, 0, rtol=0.0, atol=0.0, xb=xb, xq=xq)


@pytest.mark.parametrize("metric", [0, 1])
def test_tile_range_search(vs, metric):
    """Range search with 300 queries runs on the tiled kernel (MODE 1)."""
    xb = syn.normal_unit(8000, 96, 17, 0)
    xq = np.concatenate([xb[:150] + 0.02, syn.normal_unit(150, 96, 17, 1)]).astype(np.float32)
    radius = 0.05 if metric == 0 else 0.6
    g = vs.GpuIndexFlat(96, vs.Metric(metric), storage="f32")
    g.add(xb)
    rr = g.range_search(xq, radius)
    tiled, _ = g.prof_get("tiled")
    g.close()
    assert tiled >= 1
    lims, D, I = oracle.flat_range_search(xb, xq, radius, metric, NT)
    assert lims[-1] >= 150
    assert_range_parity(rr.limits, rr.distances, rr.ids, lims, D, I)


def test_tile_query_blocks_past_256_padding(vs, monkeypatch):
    """96-query blocks with 1,024 queries: the last block reaches query row
    1,055, past a 256-row multiple; the prepared query planes and shared
    thresholds are padded for it (regression test of that padding)."""
    monkeypatch.setenv("VS_TILE_QB", "3")
    xb16 = syn.to_bf16_bits(syn.normal_unit(6000, 768, 41, 0))
    xq16 = syn.to_bf16_bits(syn.normal_unit(1024, 768, 41, 1))
    D, I, tiled, _ = _search(vs, xb16, xq16, 10, 1, "bf16")
    assert tiled >= 1
    Dr, Ir = oracle.flat_search(syn.bf16_bits_to_f32(xb16), syn.bf16_bits_to_f32(xq16), 10, 1, NT)
    assert_knn_parity(D, I, Dr, Ir, 1, rtol=1e-3)
