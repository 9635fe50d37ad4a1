"""Config 3 at full size: 20,000,000 x 768 bf16 unit rows (30.7 GB in HBM,
15.4e9 elements, past the 2^31-element offsets that bound the reference's
engine, engine.cu:24-29), IP, k = 10, batches 1 / 64 / 1024 / 8192.

- The device generator's rows equal the host restatement of it, bit for bit.
- Stored rows past 2^31 elements, used as queries, find themselves first
  with the exact fp64 score.
- Sampled queries of every batch match the oracle (IndexFlat.search,
  index_flat.dart:62-97) run over the whole database, streamed to the host
  in chunks whose top-k lists are merged.
"""
import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity
from _philox import normalized_rows
from vector_store import synthetic as syn

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()
N, D, K, SEED, CHUNK = 20_000_000, 768, 10, 1234, 1 << 20
ROW_2_31 = (1 << 31) // D + 1  # first row whose first element lies past 2^31


@pytest.fixture(scope="module")
def c3(vs):
    idx = vs.GpuIndexFlat(D, vs.Metric.innerProduct, storage="bf16")
    syn.add_device_normal(idx, N, D, SEED, CHUNK)
    assert idx.ntotal == N and idx.storage == "bf16"
    yield idx
    idx.close()


def host_rows(rows):
    """The generator's bf16 rows, restated on the host."""
    out = []
    for r in rows:
        c0 = (r // CHUNK) * CHUNK
        v = normalized_rows([r - c0], D, SEED, syn.DEVICE_STREAM_BASE + c0)
        out.append(syn.to_bf16_bits(v)[0])
    return np.stack(out)


def test_generator_matches_host(c3):
    g = syn.rng(77, 0)
    rows = sorted({0, 1, CHUNK - 1, CHUNK, ROW_2_31 - 1, ROW_2_31, 2_800_000, 10_000_000,
                   N - CHUNK, N - 1, *g.integers(0, N, 22).tolist()})
    got = np.stack([syn.to_bf16_bits(c3.reconstruct(r)) for r in rows])
    want = host_rows(rows)
    diff = np.nonzero(np.any(got != want, axis=1))[0]
    assert diff.size == 0, f"rows {[rows[i] for i in diff[:5]]} differ from the host generator"
    # unit norm within bf16 rounding
    n2 = (syn.bf16_bits_to_f32(got).astype(np.float64) ** 2).sum(1)
    assert np.all(np.abs(n2 - 1.0) < 1e-2)


def test_rows_past_2_31_find_themselves(c3):
    rows = [ROW_2_31, ROW_2_31 + 1, 2_800_000, 5_000_003, 12_345_678, N - 2, N - 1]
    q16 = np.stack([syn.to_bf16_bits(c3.reconstruct(r)) for r in rows])
    r = c3.search(q16, K)
    assert list(r.ids[:, 0]) == rows
    x = syn.bf16_bits_to_f32(q16).astype(np.float64)
    self_ip = np.array([np.sum(v * v) for v in x]).astype(np.float32)  # fp64 sum, in order
    exact = np.array([float(np.float32(sum(float(t) * float(t) for t in v))) for v in x],
                     np.float32)
    assert np.array_equal(r.distances[:, 0], exact)
    assert np.allclose(self_ip, exact, rtol=1e-6)


@pytest.mark.timeout(900)
def test_batches_match_oracle_on_full_database(c3):
    xq16 = syn.to_bf16_bits(syn.normal_unit(8192, D, SEED, 1))
    xq = syn.bf16_bits_to_f32(xq16)
    sample = {1: [0], 64: [0, 63], 1024: [5, 1023], 8192: [4096, 8191]}
    qids = sorted({q for v in sample.values() for q in v})
    got = {}
    for B, pos in sample.items():
        r = c3.search(xq16[:B], K)
        got[B] = (r.distances[pos], r.ids[pos])
    # oracle over the whole database, chunk by chunk, merged per query
    cand_d, cand_i = [], []
    for r0 in range(0, N, CHUNK):
        rows = c3.reconstruct_n(r0, min(CHUNK, N - r0))
        Dc, Ic = oracle.flat_search(rows, xq[qids], K, oracle.IP, NT)
        cand_d.append(Dc)
        cand_i.append(np.where(Ic >= 0, Ic + r0, -1))
    cd = np.concatenate(cand_d, axis=1)
    ci = np.concatenate(cand_i, axis=1)
    Dr = np.empty((len(qids), K), np.float32)
    Ir = np.empty((len(qids), K), np.int32)
    for j in range(len(qids)):
        order = np.lexsort((ci[j], -cd[j].astype(np.float64)))[:K]
        Dr[j], Ir[j] = cd[j][order], ci[j][order]
    where = {q: j for j, q in enumerate(qids)}
    for B, pos in sample.items():
        rows = [where[q] for q in pos]
        assert_knn_parity(got[B][0], got[B][1], Dr[rows], Ir[rows], 1, rtol=1e-3)
