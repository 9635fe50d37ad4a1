"""The bench harness mirror (vector_store/bench.py) against the reference's
own harness tests (test/vector_store_test.dart:2750-2930): recall of the
flat baseline, sweep rows, RFC-4180 CSV, GFM Markdown, Pareto frontier,
argument checks.  The index here is a small numpy flat index (host logic
only); tests/test_gpu_bench_harness.py runs it on the GPU index beside the
CPU oracle, as bench_faiss.dart's four flat rows."""
import numpy as np
import pytest

from vector_store import SearchResult
from vector_store.bench import (BenchOptions, BenchResult, bench_index, bench_index_sweep,
                                dart_fixed, format_bench_table, pareto_frontier, to_bench_csv,
                                to_bench_markdown)


class NumpyFlatL2:
    def __init__(self, xb):
        self.xb = np.asarray(xb, np.float32)

    @property
    def ntotal(self):
        return len(self.xb)

    def search(self, q, k):
        d = ((np.asarray(q, np.float64)[:, None, :] - self.xb[None].astype(np.float64)) ** 2).sum(-1)
        order = np.argsort(d, axis=1, kind="stable")[:, :k]
        return SearchResult(np.take_along_axis(d, order, 1).astype(np.float32),
                            order.astype(np.int32))


class DropFirst(NumpyFlatL2):
    """Misses every query's best neighbour (a lossy index)."""

    def search(self, q, k):
        r = super().search(q, k + 1)
        return SearchResult(r.distances[:, 1:], r.ids[:, 1:])


@pytest.fixture
def data():
    g = np.random.default_rng(3)
    xs = g.standard_normal((300, 8)).astype(np.float32)
    qs = g.standard_normal((12, 8)).astype(np.float32)
    flat = NumpyFlatL2(xs)
    return flat, qs, flat.search(qs, 5)


def test_flat_baseline_recall_is_one(data):
    flat, qs, truth = data
    r = bench_index(flat, qs, 5, truth, label="flat",
                    options=BenchOptions(warmup=0, repeats=1, per_query=False))
    assert (r.label, r.nq, r.k, r.ntotal) == ("flat", 12, 5, 300)
    assert r.recall == 1.0 and r.mean_us >= 0.0
    r = bench_index(flat, qs, 5, truth)  # per-query, warmup 1, repeats 3
    assert r.recall == 1.0 and r.p50_us <= r.p95_us <= r.p99_us


def test_recall_degrades_on_a_lossy_index(data):
    flat, qs, truth = data
    r = bench_index(DropFirst(flat.xb), qs, 5, truth, options=BenchOptions(warmup=0, repeats=1))
    assert 0.0 < r.recall < 1.0
    assert r.recall == pytest.approx(4 / 5)


def test_sweep_one_row_per_value(data):
    flat, qs, truth = data
    rows = bench_index_sweep(flat, qs, 5, truth, [1, 4, 16], lambda v: f"np={v}",
                             options=BenchOptions(warmup=0, repeats=1))
    assert [r.label for r in rows] == ["np=1", "np=4", "np=16"]


def test_csv_rfc4180():
    row = BenchResult("x, \"hi\"", 10, 5, 0.5, 12.0, 10.0, 20.0, 25.0, 100)
    lines = to_bench_csv([row]).strip().split("\n")
    assert len(lines) == 2
    assert lines[0] == "label,ntotal,nq,k,recall,mean_us,p50_us,p95_us,p99_us"
    assert lines[1].startswith('"x, ""hi"""')
    assert lines[1] == '"x, ""hi""",100,10,5,0.500000,12.000,10.000,20.000,25.000'


def test_markdown_right_aligned_escaped():
    row = BenchResult("a|b\\c", 1, 1, 0.9, 12.5, 10.0, 20.0, 30.0, 5)
    lines = to_bench_markdown([row]).strip().split("\n")
    assert len(lines) == 3
    assert lines[0].startswith("| label |") and "---:" in lines[1]
    assert "a\\|b\\\\c" in lines[2] and lines[2].endswith("| 1 |")
    assert lines[2] == "| a\\|b\\\\c | 0.900 | 12.5 | 10.0 | 20.0 | 30.0 | 5 | 1 | 1 |"


def test_table_and_fixed_rounding():
    assert dart_fixed(1.0625, 3) == "1.063"  # half away from zero, as toStringAsFixed
    assert dart_fixed(0.5, 0) == "1" and dart_fixed(2.675, 2) == "2.67"  # 2.675 is below .675
    t = format_bench_table([BenchResult("flat", 4, 2, 1.0, 3.25, 3.0, 4.0, 5.0, 9)])
    assert t.splitlines()[0].startswith("label       ")
    assert format_bench_table([]) == "(no rows)\n"


def _row(label, recall, mean):
    return BenchResult(label, 1, 1, recall, mean, mean, mean, mean, 100)


def test_pareto_frontier():
    rows = [_row("fast-lowrecall", 0.2, 5), _row("dominated", 0.3, 25),
            _row("mid-mediocre", 0.5, 10), _row("slow-perfect", 1.0, 100)]
    assert [r.label for r in pareto_frontier(rows)] == ["fast-lowrecall", "mid-mediocre",
                                                        "slow-perfect"]
    tie = pareto_frontier([_row("slow-recall1", 1.0, 100), _row("fast-recall1", 1.0, 50)])
    assert [r.label for r in tie] == ["fast-recall1"]
    assert pareto_frontier([]) == []


def test_rejects_mismatched_truth(data):
    flat, qs, truth = data
    with pytest.raises(ValueError):
        bench_index(flat, qs[:3], 5, truth)
    with pytest.raises(ValueError):
        bench_index(flat, qs, truth.k + 1, truth)
    with pytest.raises(ValueError):
        bench_index(flat, qs[:0], 5, truth)
