"""Recall / latency harness of the vector store (lib/core/vector_store/bench.dart).

Same names, arguments and rules as the reference:

- bench_index (benchIndex, bench.dart:90-184): `warmup` discarded passes, then
  `repeats` timed passes; per-query mode times one search([q], k) call per
  query, batched mode times one call and spreads it evenly over the queries;
  the pass with the smallest total is kept, and mean / p50 / p95 / p99 are
  taken from it with the nearest-rank index round((n - 1) q);
- recall_at_k (_recallAtK, bench.dart:356-371): |result ∩ truth| / (nq k),
  truth ids of -1 are not gold;
- to_bench_csv / format_bench_table / to_bench_markdown (bench.dart:221-312)
  and pareto_frontier (bench.dart:314-350) produce the same text.

Times are microseconds of host wall clock around each search call, as the
reference's Stopwatch measures them (so they include the library call and,
for host buffers, the PCIe transfers).
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass
from decimal import ROUND_HALF_UP, Decimal
from typing import Callable, Iterable, List, Sequence

import numpy as np

from .index import SearchResult, recall_at_k


def dart_fixed(x: float, digits: int) -> str:
    """double.toStringAsFixed: the exact binary value rounded half away from zero."""
    if math.isnan(x):
        return "NaN"
    if math.isinf(x):
        return "Infinity" if x > 0 else "-Infinity"
    q = Decimal(1).scaleb(-digits)
    return format(Decimal(x).quantize(q, rounding=ROUND_HALF_UP), "f")


@dataclass
class BenchResult:
    """bench.dart:19-68."""

    label: str
    nq: int
    k: int
    recall: float
    mean_us: float
    p50_us: float
    p95_us: float
    p99_us: float
    ntotal: int

    def __str__(self) -> str:
        return (f"BenchResult({self.label}: recall@{self.k}={dart_fixed(self.recall, 3)}, "
                f"mean={dart_fixed(self.mean_us, 1)}µs, p50={dart_fixed(self.p50_us, 1)}µs, "
                f"p95={dart_fixed(self.p95_us, 1)}µs, ntotal={self.ntotal}, nq={self.nq})")


@dataclass(frozen=True)
class BenchOptions:
    """bench.dart:70-87: warmup passes, timed repeats, per-query timing."""

    warmup: int = 1
    repeats: int = 3
    per_query: bool = True


def _round_half_away(x: float) -> int:
    return int(math.floor(x + 0.5)) if x >= 0 else -int(math.floor(-x + 0.5))


def _pct(sorted_us: Sequence[int], q: float) -> float:
    if not sorted_us:
        return 0.0
    return float(sorted_us[_round_half_away((len(sorted_us) - 1) * q)])


def bench_index(index, queries, k: int, truth: SearchResult, label: str = "index",
                options: BenchOptions = BenchOptions()) -> BenchResult:
    """benchIndex (bench.dart:90-184)."""
    q = np.asarray(queries)
    nq = int(q.shape[0]) if q.ndim == 2 else len(queries)
    if nq == 0:
        raise ValueError("benchIndex: queries is empty")
    if truth.nq != nq:
        raise ValueError(f"benchIndex: truth.nq={truth.nq} != queries.length={nq}")
    if truth.k < k:
        raise ValueError(f"benchIndex: truth.k={truth.k} is smaller than requested k={k}")
    for _ in range(options.warmup):
        index.search(q, k)
    best_total = 1 << 62
    best_us: List[int] = []
    best_res = None
    for _ in range(options.repeats):
        pass_us = [0] * nq
        if options.per_query:
            D = np.empty((nq, k), np.float32)
            I = np.empty((nq, k), np.int32)
            total = 0
            for qi in range(nq):
                t0 = time.perf_counter_ns()
                one = index.search(q[qi:qi + 1], k)
                us = (time.perf_counter_ns() - t0) // 1000
                pass_us[qi] = us
                total += us
                D[qi], I[qi] = one.distances[0], one.ids[0]
            res = SearchResult(D, I)
        else:
            t0 = time.perf_counter_ns()
            res = index.search(q, k)
            total = (time.perf_counter_ns() - t0) // 1000
            per = _round_half_away(total / nq)
            pass_us = [per] * nq
        if total < best_total:
            best_total, best_us, best_res = total, pass_us, res
    srt = sorted(best_us)
    return BenchResult(label=label, nq=nq, k=k, recall=recall_at_k(best_res, truth, k),
                       mean_us=sum(best_us) / len(best_us), p50_us=_pct(srt, 0.5),
                       p95_us=_pct(srt, 0.95), p99_us=_pct(srt, 0.99), ntotal=int(index.ntotal))


def bench_index_sweep(index, queries, k: int, truth: SearchResult, values: Iterable,
                      configure: Callable[[object], str],
                      options: BenchOptions = BenchOptions()) -> List[BenchResult]:
    """benchIndexSweep (bench.dart:186-215): one row per value, in order."""
    out = []
    for v in values:
        label = configure(v)
        out.append(bench_index(index, queries, k, truth, label=label, options=options))
    return out


def _csv_escape(s: str) -> str:
    if "," in s or '"' in s or "\n" in s:
        return '"' + s.replace('"', '""') + '"'
    return s


def _md_escape(s: str) -> str:
    return s.replace("\\", "\\\\").replace("|", "\\|").replace("\r\n", "<br>").replace("\n", "<br>")


def to_bench_csv(rows: Iterable[BenchResult]) -> str:
    """toBenchCsv (bench.dart:217-245)."""
    out = ["label,ntotal,nq,k,recall,mean_us,p50_us,p95_us,p99_us\n"]
    for r in rows:
        out.append(",".join([_csv_escape(r.label), str(r.ntotal), str(r.nq), str(r.k),
                             dart_fixed(r.recall, 6), dart_fixed(r.mean_us, 3),
                             dart_fixed(r.p50_us, 3), dart_fixed(r.p95_us, 3),
                             dart_fixed(r.p99_us, 3)]) + "\n")
    return "".join(out)


def format_bench_table(rows: Iterable[BenchResult]) -> str:
    """formatBenchTable (bench.dart:247-277): fixed-width text."""
    rows = list(rows)
    if not rows:
        return "(no rows)\n"
    lw = max(12, max(len(r.label) for r in rows))
    out = [r"label".ljust(lw),
           "  recall   mean_us    p50_us    p95_us    p99_us  ntotal   nq   k\n",
           "-" * (lw + 68) + "\n"]
    for r in rows:
        out += [r.label.ljust(lw), "  ", dart_fixed(r.recall, 3).rjust(7),
                dart_fixed(r.mean_us, 1).rjust(10), dart_fixed(r.p50_us, 1).rjust(10),
                dart_fixed(r.p95_us, 1).rjust(10), dart_fixed(r.p99_us, 1).rjust(10),
                str(r.ntotal).rjust(8), str(r.nq).rjust(5), str(r.k), "\n"]
    return "".join(out)


def to_bench_markdown(rows: Iterable[BenchResult]) -> str:
    """toBenchMarkdown (bench.dart:279-312)."""
    out = ["| label | recall | mean_us | p50_us | p95_us | p99_us | ntotal | nq | k |\n"
           "| :--- | ---: | ---: | ---: | ---: | ---: | ---: | ---: | ---: |\n"]
    for r in rows:
        out.append("| " + " | ".join([_md_escape(r.label), dart_fixed(r.recall, 3),
                                      dart_fixed(r.mean_us, 1), dart_fixed(r.p50_us, 1),
                                      dart_fixed(r.p95_us, 1), dart_fixed(r.p99_us, 1),
                                      str(r.ntotal), str(r.nq), str(r.k)]) + " |\n")
    return "".join(out)


def pareto_frontier(rows: Iterable[BenchResult]) -> List[BenchResult]:
    """paretoFrontier (bench.dart:314-350): the rows no other row beats on both
    recall and mean_us, recall ascending; on recall ties the fastest (first in
    input order among equals) survives."""
    inp = list(rows)
    if not inp:
        return []
    # a stable sort: recall descending, then mean_us ascending
    srt = sorted(inp, key=lambda r: (-r.recall, r.mean_us))
    out = []
    best_us = math.inf
    last_recall = None
    for r in srt:
        if r.recall == last_recall:
            continue
        if r.mean_us < best_us:
            out.append(r)
            best_us = r.mean_us
            last_recall = r.recall
    return list(reversed(out))
