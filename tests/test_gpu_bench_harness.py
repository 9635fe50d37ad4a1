"""benchIndex (bench.dart:90-184) on the GPU index, as bench_faiss.dart:55-103
runs its four flat rows: the CPU IndexFlat (the oracle, timed by the same
harness) and GpuIndexFlat, each per query and batched, against the oracle's
ground truth; then the rows through toBenchCsv / toBenchMarkdown
(bench.dart:221-312)."""
import numpy as np
import pytest

import oracle
from vector_store import SearchResult
from vector_store import synthetic as syn
from vector_store.bench import BenchOptions, bench_index, to_bench_csv, to_bench_markdown

pytestmark = pytest.mark.gpu
NT = oracle.default_threads()


def labels(metric):
    cpu = "IndexFlatL2" if metric == 0 else "IndexFlatIP"
    return [cpu, "GpuIndexFlat", cpu + " [batched]", "GpuIndexFlat [batched]"]


def _rows(vs, metric, storage, xb, xq, k):
    idx = vs.GpuIndexFlat(xb.shape[1], vs.Metric(metric), storage=storage)
    idx.add(xb)
    Dt, It = oracle.flat_search(xb, xq, k, metric, NT)
    truth = SearchResult(Dt, It)
    cpu = oracle.FlatIndex(xb, metric, NT)
    batched = BenchOptions(per_query=False)
    lab = labels(metric)
    rows = [bench_index(cpu, xq, k, truth, label=lab[0]),
            bench_index(idx, xq, k, truth, label=lab[1]),
            bench_index(cpu, xq, k, truth, label=lab[2], options=batched),
            bench_index(idx, xq, k, truth, label=lab[3], options=batched)]
    n = idx.ntotal
    idx.close()
    return rows, n


@pytest.mark.parametrize("metric,storage", [(0, "f32"), (1, "bf16"), (0, "auto")])
def test_bench_faiss_flat_rows(vs, metric, storage):
    if storage == "auto":  # configs[1] arithmetic: integers 0..255, kept losslessly as bf16
        xb, xq = syn.int_grid(20_000, 128, 7, 0), syn.int_grid(48, 128, 7, 1)
    else:
        xb, xq = syn.normal_unit(20_000, 96, 7, 0), syn.normal_unit(48, 96, 7, 1)
        if storage == "bf16":
            xb = syn.bf16_bits_to_f32(syn.to_bf16_bits(xb))
    k = 10
    rows, n = _rows(vs, metric, storage, xb, xq, k)
    for r in rows:
        # the GPU rows find exactly the oracle's neighbours; so does the
        # oracle itself (its own truth)
        assert r.recall == 1.0, r
        assert r.nq == len(xq) and r.k == k and r.ntotal == n
        assert 0 <= r.p50_us <= r.p95_us <= r.p99_us
        assert r.mean_us >= 0
    assert rows[0].mean_us > 0 and rows[1].mean_us > 0  # per-query calls take time
    # batched rows spread one call's time evenly over the queries
    for r in rows[2:]:
        assert r.p50_us == r.p95_us == r.p99_us
    csv = to_bench_csv(rows).splitlines()
    assert len(csv) == 5 and csv[0].startswith("label,")
    assert [line.split(",")[0] for line in csv[1:]] == labels(metric)
    md = to_bench_markdown(rows).splitlines()
    assert [line.split(" | ")[0][2:] for line in md[2:]] == labels(metric)


def test_bench_index_recall_counts_misses(vs):
    """Recall below 1 when the truth asks for neighbours the index cannot
    return (k > ntotal pads with id -1, which never matches a gold id)."""
    xb = syn.normal_unit(300, 32, 9, 0)
    xq = syn.normal_unit(8, 32, 9, 1)
    idx = vs.GpuIndexFlat.l2(32, storage="f32")
    idx.add(xb[:5])
    Dt, It = oracle.flat_search(xb, xq, 10, 0, NT)
    r = bench_index(idx, xq, 10, SearchResult(Dt, It), label="GpuIndexFlat",
                    options=BenchOptions(warmup=0, repeats=1))
    idx.close()
    gold = sum(len(set(It[q].tolist()) & set(range(5))) for q in range(len(xq)))
    assert r.recall == gold / (len(xq) * 10) < 1.0
