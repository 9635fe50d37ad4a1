"""Benchmark of the MI355X flat k-NN path (one JSON line on stdout).

Default run (no flags): every BASELINE.json configuration, in one process.
The headline line is configs[1] (C2): exact L2 top-100 over a 1,000,000 x 128
database of integers 0..255 stored as fp32, 10,000 queries of the same
distribution; one step = one search of the whole query batch with the
database, the queries and the result buffers resident in HBM.  The other
configurations sit under "workloads":

  c1  10k x 384 fp32 unit rows, IP, 100 queries, k = 10 (the CPU-runnable case);
  c2f configs[1]'s shape on fp32 unit N(0,1) rows, which bf16 does not hold
      exactly: the rows stay fp32 and every product takes three MFMA passes
      over split-bf16 planes (the path of general fp32 embeddings);
  c3  20M x 768 bf16 unit rows (device-generated), IP, k = 10, batches
      1 / 64 / 1024 / 8192;
  c4  k-means step, 2M x 256 fp32 mixture points, K = 4096;
  c5  cosine self-join of 500k x 512 fp32 unit rows, threshold 0.95.

Every workload reports:
  value / ms_per_step   whole-job rate over the K timed steps (inputs in HBM);
  steps_ms              best / median / p50 / p95 / p99 of the step times
                        (the benchIndex protocol, bench.dart:90-184: warmup,
                        repeated timed passes, best and median);
  roofline              the dominant kernel timed with HIP events on the
                        index's stream over the timed region: algorithmic
                        bytes (HBM-bound: batch <= 64) or flops (MFMA-bound)
                        per launch over its mean duration, against the spec
                        peak and against the measured peaks (vs_dev_probe);
  cpu_baseline          the CPU oracle (oracle/oracle.c, a restatement of
                        IndexFlat.search / rangeSearch / Kmeans, index_flat.dart,
                        kmeans.dart) timed on this host: all cores (threads
                        over queries, at most the box's 16-core share) and one
                        core (the reference's own parallelism: one Dart isolate);
  parity                GPU results against the oracle on the same inputs:
                        tie-aware top-k comparison (distances bit-identical,
                        ids equal outside exact-tie groups), identical k-means
                        assignments and centroids, identical pair lists.

C2 also reports the PCIe-inclusive rate of the host-buffer entry point
(vs_index_search) and benchIndex rows in the reference's CSV / Markdown
formats (toBenchCsv / toBenchMarkdown, bench.dart:217-312); --csv / --md write
them to files.

Single workloads (--workload c1|c2|c2f|c3|c4|c5, --batch for c3) print that
workload's line alone (profiling runs use them); --workload copy / libgemm are
the counter yardstick and the vendor GEMM for scale.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "dart-pytorch_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "QPS, flat top-k k-NN (1M×128 fp32, 20M×768 bf16); % HBM / MFMA roofline"
PEAK = {"bf16_mfma_tflops": 2500.0, "fp32_mfma_tflops": 157.3, "hbm_gbs": 8000.0}
CPU_SHARE = 16  # host cores of one GPU's share on the measurement boxes

# HBM bytes per launch of the dominant kernel, from two rocprofv3 --pmc runs
# (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0: the factors a plain 16-byte copy of
# known size reads, profiles/copy16_calibration.md), keyed by
# (workload, n, nq, k).  The command and readings are in the named profile;
# configurations without a measurement report traffic null.
MEASURED_TRAFFIC = {
    ("c2", 1_000_000, 10_000, 100): (1.199e9, "profiles/scan_c2_1Mx128_k100.md"),
    ("c3", 20_000_000, 1, 10): (30.73e9, "profiles/scan_c3_20Mx768_b1_b64.md"),
    ("c3", 20_000_000, 64, 10): (30.78e9, "profiles/scan_c3_20Mx768_b1_b64.md"),
    ("c3", 20_000_000, 1024, 10): (31.94e9, "profiles/gemm_c3_20Mx768_b1024_b8192.md"),
    ("c3", 20_000_000, 8192, 10): (325.3e9, "profiles/gemm_c3_20Mx768_b1024_b8192.md"),
    ("c4", 2_000_000, 4096, 256): (2.38e9, "profiles/kmeans_c4_2Mx256.md"),
    ("c5", 500_000, 500_000, 512): (278.25e9, "profiles/selfjoin_c5_500kx512.md"),
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# --------------------------------------------------------------------------
# host facts, peaks, timing statistics
# --------------------------------------------------------------------------
def host_info():
    cpu, mem, ident = "unknown", None, {}
    try:
        for line in open("/proc/cpuinfo"):
            key = line.split(":", 1)[0].strip()
            if key in ("model name", "cpu family", "model", "stepping", "cpu MHz") and key not in ident:
                ident[key] = line.split(":", 1)[1].strip()
            if key == "processor" and ident:
                break
        cpu = ident.get("model name", cpu)
        for line in open("/proc/meminfo"):
            if line.startswith("MemTotal"):
                mem = round(int(line.split()[1]) / 2 ** 20, 1)
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    return {"cpu_model": cpu, "cpu_family_model_stepping": [ident.get("cpu family"),
                                                               ident.get("model"),
                                                               ident.get("stepping")],
            "cpu_mhz": ident.get("cpu MHz"), "nproc": os.cpu_count(), "affinity_cores": affinity,
            "mem_gib": mem, "threads_all_core": max(1, min(affinity, CPU_SHARE))}


def measured_peaks(NN):
    """Achievable read bandwidth and bf16 MFMA rate on this GPU (vs_dev_probe)."""
    import ctypes

    out = {}
    for what, key, nbytes in ((0, "hbm_read_gbs", 8 << 30), (1, "bf16_mfma_tflops", 0),
                              (2, "bf16_mfma_random_tflops", 0)):
        v = ctypes.c_double(0.0)
        rc = NN.load().vs_dev_probe(0, what, nbytes, ctypes.byref(v))
        out[key] = round(v.value, 1) if rc == 0 else None
    return out


def step_stats(times_s):
    t = np.sort(np.asarray(times_s) * 1e3)
    n = len(t)

    def pct(q):  # nearest rank, as benchIndex (bench.dart:167-171)
        return float(t[int(np.floor((n - 1) * q + 0.5))])

    return {"best_ms": round(float(t[0]), 4), "median_ms": round(float(np.median(t)), 4),
            "mean_ms": round(float(t.mean()), 4), "p50_ms": round(pct(0.5), 4),
            "p95_ms": round(pct(0.95), 4), "p99_ms": round(pct(0.99), 4), "n": n}


def time_steps(fn, steps, warmup, label):
    for _ in range(warmup):
        fn()
    times = []
    t0 = time.perf_counter()
    for i in range(steps):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    wall = time.perf_counter() - t0
    log(f"[bench] {label}: {steps} steps in {wall:.3f} s")
    return wall, times


def roofline(kind, work, avg_s, peaks, kernel, launches, traffic=None, traffic_src=None,
             peak_div=1, extra=None):
    """kind 'hbm': work = algorithmic bytes per launch; 'mfma': flops per launch."""
    if kind == "hbm":
        ach = work / avg_s / 1e9
        peak, meas, unit = PEAK["hbm_gbs"], peaks.get("hbm_read_gbs"), "GB/s"
    else:
        ach = work / avg_s / 1e12
        peak = PEAK["bf16_mfma_tflops"] / peak_div
        m = peaks.get("bf16_mfma_tflops")
        meas, unit = (m / peak_div if m else None), "TFLOP/s"
        mr = peaks.get("bf16_mfma_random_tflops")
        mr = mr / peak_div if mr else None
    r = {"bound": kind, "achieved": round(ach, 2), "peak": round(peak, 1), "unit": unit,
         "frac": round(ach / peak, 4), "traffic": traffic,
         "measured_peak": round(meas, 1) if meas else None,
         "frac_of_measured": round(ach / meas, 4) if meas else None,
         **({} if kind == "hbm" else {
             "measured_peak_random": round(mr, 1) if mr else None,
             "frac_of_measured_random": round(ach / mr, 4) if mr else None}),
         "kernel": kernel, "launches": launches, "avg_ms": round(avg_s * 1e3, 4),
         ("algorithmic_bytes_per_launch" if kind == "hbm" else "algorithmic_flops_per_launch"): work}
    if traffic_src:
        r["traffic_source"] = traffic_src
    if extra:
        r.update(extra)
    return r


def kernel_avg(idx, fam):
    n, ms = idx.prof_get(fam)
    return n, (ms / max(n, 1)) / 1e3


def mfma_passes(idx):
    """bf16 MFMA passes per distance of an fp32-row scan: 1 when the one-pass
    bf16 selection ran (GEMM shapes of storage code 2, or 1 on the bf16 copy
    of the rows, or the row-shared scan, which reads fp32 rows only that
    way), else 3 (hi*q0 + lo*q0 + hi*q1 of the split-bf16 planes)."""
    coarse = sum(idx.prof_get(f"gemm:{st},1,2,{wq},4,2,{kc}")[0]
                 for st in (1, 2) for wq in (2, 4) for kc in (32, 64))
    coarse += idx.prof_get("gemm:1,1,2,2,4,4,32")[0]  # the four-wave kernel on the bf16 copy
    coarse += idx.prof_get("shared")[0]
    return 1 if coarse else 3


# --------------------------------------------------------------------------
# CPU oracle timing
# --------------------------------------------------------------------------
def cpu_search(xb, xq, k, metric, threads, target_s):
    """The oracle on a bounded query sample of the batch: (qps, queries, seconds, (D, I))."""
    import oracle

    n0 = min(len(xq), max(threads, 1))
    t = time.perf_counter()
    oracle.flat_search(xb, xq[:n0], k, metric, threads)
    per_q = (time.perf_counter() - t) / n0
    ns = int(min(len(xq), max(n0, target_s / max(per_q, 1e-9))))
    if ns >= threads:
        ns = (ns // threads) * threads
    t = time.perf_counter()
    D, I = oracle.flat_search(xb, xq[:ns], k, metric, threads)
    dt = time.perf_counter() - t
    return ns / dt, ns, dt, (D, I)


def cpu_baseline_entry(all_core, one_core, unit, sample, host):
    qa, na, ta = all_core
    out = {"value": round(qa, 3), "unit": unit, "cores": host["threads_all_core"], "kind": "port",
           "sample": sample.format(n=na, t=ta), "cpu": host["cpu_model"], "nproc": host["nproc"]}
    if one_core is not None:
        q1, n1, t1 = one_core
        out["single_core"] = {"value": round(q1, 3), "unit": unit, "cores": 1,
                              "sample": sample.format(n=n1, t=t1)}
    return out


# --------------------------------------------------------------------------
# C1 / C2: flat search with host-generated inputs
# --------------------------------------------------------------------------
def search_setup(vs, NN, workload, args):
    from vector_store import synthetic as syn

    if workload == "c2":
        n, d, nq, k, metric = args.n or 1_000_000, 128, args.nq or 10_000, args.k or 100, 0
        xb, xq = syn.int_grid(n, d, args.seed, 0), syn.int_grid(nq, d, args.seed, 1)
        storage = "auto"
        desc = f"c2: exact L2 top-{k}, {n} x {d} fp32 integers 0..255, {nq} queries"
    elif workload == "c2f":
        # configs[1]'s shape on general fp32 values (not exact in bf16): the rows stay fp32
        # and the scan multiplies their split-bf16 planes, three MFMA passes per product
        n, d, nq, k, metric = args.n or 1_000_000, 128, args.nq or 10_000, args.k or 100, 0
        xb, xq = syn.normal_unit(n, d, args.seed, 0), syn.normal_unit(nq, d, args.seed, 1)
        storage = "auto"
        desc = (f"c2 shape on fp32 data: exact L2 top-{k}, {n} x {d} fp32 unit N(0,1), "
                f"{nq} queries (split-bf16 planes, three MFMA passes)")
    else:
        n, d, nq, k, metric = args.n or 10_000, 384, args.nq or 100, args.k or 10, 1
        xb, xq = syn.normal_unit(n, d, args.seed, 0), syn.normal_unit(nq, d, args.seed, 1)
        storage = "f32"
        desc = f"c1: exact IP top-{k}, {n} x {d} fp32 unit N(0,1), {nq} queries"
    return n, d, nq, k, metric, xb, xq, storage, desc


def run_search(vs, NN, workload, args, ctx, full=False):
    import oracle
    from oracle.parity import knn_failures

    n, d, nq, k, metric, xb, xq, storage, desc = search_setup(vs, NN, workload, args)
    idx = vs.GpuIndexFlat(d, vs.Metric(metric), storage=storage)
    idx.add(xb)
    qbuf = NN.DeviceBuffer(xq.nbytes)
    qbuf.upload(xq)
    Dbuf, Ibuf = NN.DeviceBuffer(nq * k * 4), NN.DeviceBuffer(nq * k * 4)

    def step():
        idx.search_device(qbuf, nq, k, Dbuf, Ibuf, NN.VS_DTYPE_F32)

    for _ in range(args.warmup):
        step()
    idx.prof_enable(True)
    idx.prof_reset()
    wall, times = time_steps(step, args.steps, 0, desc)
    idx.prof_enable(False)
    nscan, scan_s = kernel_avg(idx, "scan")
    nmerge, merge_s = kernel_avg(idx, "merge")
    npre, pre_ms = idx.prof_get("prepass")
    D = np.empty((nq, k), np.float32)
    I = np.empty((nq, k), np.int32)
    Dbuf.download(D)
    Ibuf.download(I)
    bf16 = idx.storage == "bf16"
    traffic, tsrc = MEASURED_TRAFFIC.get((workload, n, nq, k), (None, None))
    roof = roofline("mfma", 2.0 * nq * n * d, scan_s, ctx["peaks"], "scan", nscan, traffic, tsrc,
                    peak_div=1 if bf16 else 3,
                    extra={"scan_kinds": {f: idx.prof_get(f)[0] for f in
                                          ("shared", "gemm", "streamed")
                                          if idx.prof_get(f)[0]},
                           "merge_avg_ms": round(merge_s * 1e3, 4),
                           "prepass_ms_per_step": round(pre_ms / args.steps, 4) if npre else None,
                           "exact_fallback_queries": idx.prof_get("exact_fallback")[0]})
    out = {"metric": METRIC, "value": round(nq * args.steps / wall, 1), "unit": "queries/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16" if bf16 else "fp32",
           "data": "synthetic", "config": {"workload": desc, "n": n, "d": d, "nq": nq, "k": k,
                                           "metric": "L2" if metric == 0 else "IP",
                                           "storage": idx.storage},
           "steps_ms": step_stats(times), "roofline": roof}

    if full:
        # PCIe-inclusive rate of the host-buffer entry point (never `value`)
        wall_h, _ = time_steps(lambda: idx.search(xq, k), max(3, args.steps // 2), 1,
                               f"{workload} host buffers")
        out["host_buffer_qps"] = round(nq * max(3, args.steps // 2) / wall_h, 1)
        # benchIndex rows (bench.dart:90-184) on query subsets with oracle truth
        from vector_store import SearchResult
        from vector_store.bench import (BenchOptions, bench_index, to_bench_csv,
                                        to_bench_markdown)

        # bench_faiss.dart:55-103's four flat rows on one query set: the CPU
        # IndexFlat (the oracle on all host threads; a single query runs on
        # one) and GpuIndexFlat, per query and batched
        th = ctx["host"]["threads_all_core"]
        nb = min(nq, 32)
        Dt, It = oracle.flat_search(xb, xq[:nb], k, metric, th)
        truth = SearchResult(Dt, It)
        cpu = oracle.FlatIndex(xb, metric, th)
        cname = "IndexFlatL2" if metric == 0 else "IndexFlatIP"
        per, bat = BenchOptions(warmup=1, repeats=3), BenchOptions(warmup=1, repeats=3,
                                                                   per_query=False)
        rows = [bench_index(cpu, xq[:nb], k, truth, label=cname, options=per),
                bench_index(idx, xq[:nb], k, truth, label="GpuIndexFlat", options=per),
                bench_index(cpu, xq[:nb], k, truth, label=cname + " [batched]", options=bat),
                bench_index(idx, xq[:nb], k, truth, label="GpuIndexFlat [batched]",
                            options=bat)]
        out["bench_index"] = [r.__dict__ for r in rows]
        out["bench_csv"] = to_bench_csv(rows)
        out["bench_markdown"] = to_bench_markdown(rows)
        ctx["bench_rows"] = rows

    if not args.no_cpu:
        host = ctx["host"]
        th = host["threads_all_core"]
        qa, na, ta, (Dc, Ic) = cpu_search(xb, xq, k, metric, th, args.cpu_seconds)
        one = None
        if not args.no_single_core:
            q1, n1, t1, _ = cpu_search(xb, xq, k, metric, 1, args.cpu_seconds / 2)
            one = (q1, n1, t1)
        out["cpu_baseline"] = cpu_baseline_entry(
            (qa, na, ta), one, "queries/s",
            "first {n} of the " + f"{nq} queries against the full {n}-row database " + "({t:.1f} s), fp64 oracle",
            host)
        bad = knn_failures(D[:na], I[:na], Dc, Ic, metric, rtol=1e-5)
        out["parity"] = {"ok": not bad, "checked_queries": int(na), "failures": len(bad),
                         "rule": "tie-aware top-k vs the oracle: distances bit-identical, ids "
                                 "equal outside exact ties (rel 1e-5)",
                         "first_failures": [str(b)[:200] for b in bad[:3]]}
    qbuf.free()
    Dbuf.free()
    Ibuf.free()
    idx.close()
    return out


# --------------------------------------------------------------------------
# C3: 20M x 768 bf16, batches 1 / 64 / 1024 / 8192
# --------------------------------------------------------------------------
C3_SAMPLE = [0, 1, 31, 63, 100, 511, 777, 1023, 2048, 3333, 4095, 4096, 6000, 7777, 8190, 8191]


def run_c3(vs, NN, args, ctx, batches):
    import oracle
    from oracle.parity import knn_failures
    from vector_store import synthetic as syn

    n, d, k = args.n or 20_000_000, 768, args.k or 10
    t0 = time.perf_counter()
    idx = vs.GpuIndexFlat(d, vs.Metric.innerProduct, storage="bf16")
    syn.add_device_normal(idx, n, d, args.seed)
    log(f"[bench] c3: {n} x {d} bf16 rows generated on the device in "
        f"{time.perf_counter() - t0:.1f} s")
    bmax = max(batches)
    xq16 = syn.to_bf16_bits(syn.normal_unit(bmax, d, args.seed, 1))
    qbuf = NN.DeviceBuffer(xq16.nbytes)
    qbuf.upload(xq16)
    Dbuf, Ibuf = NN.DeviceBuffer(bmax * k * 4), NN.DeviceBuffer(bmax * k * 4)
    per_batch = {}
    results = {}
    for B in batches:
        def step():
            idx.search_device(qbuf, B, k, Dbuf, Ibuf, NN.VS_DTYPE_BF16)

        for _ in range(args.warmup):
            step()
        idx.prof_enable(True)
        idx.prof_reset()
        wall, times = time_steps(step, args.steps, 0, f"c3 batch {B}")
        idx.prof_enable(False)
        nscan, scan_s = kernel_avg(idx, "scan")
        npre, pre_ms = idx.prof_get("prepass")
        nmerge, merge_s = kernel_avg(idx, "merge")
        D = np.empty((B, k), np.float32)
        I = np.empty((B, k), np.int32)
        Dbuf.download(D)
        Ibuf.download(I)
        pos = [p for p in C3_SAMPLE if p < B]
        results[B] = (D[pos], I[pos], pos)
        traffic, tsrc = MEASURED_TRAFFIC.get(("c3", n, B, k), (None, None))
        extra = {"scan_kinds": {f: idx.prof_get(f)[0] for f in ("shared", "gemm", "streamed")
                                if idx.prof_get(f)[0]},
                 "merge_avg_ms": round(merge_s * 1e3, 4),
                 "prepass_ms_per_step": round(pre_ms / args.steps, 4) if npre else None,
                 "exact_fallback_queries": idx.prof_get("exact_fallback")[0]}
        if B <= 64:
            roof = roofline("hbm", n * d * 2, scan_s, ctx["peaks"], "scan", nscan, traffic, tsrc,
                            extra=extra)
            roof["step_frac"] = round(n * d * 2 / (wall / args.steps) / 1e9 / PEAK["hbm_gbs"], 4)
        else:
            roof = roofline("mfma", 2.0 * B * n * d, scan_s, ctx["peaks"], "scan", nscan, traffic,
                            tsrc, extra=extra)
            roof["step_frac"] = round(2.0 * B * n * d / (wall / args.steps) / 1e12 /
                                      PEAK["bf16_mfma_tflops"], 4)
        per_batch[str(B)] = {"value": round(B * args.steps / wall, 1), "unit": "queries/s",
                             "ms_per_step": round(wall / args.steps * 1e3, 3),
                             "steps_ms": step_stats(times), "roofline": roof}
    out = {"config": {"workload": f"c3: exact IP top-{k}, {n} x {d} bf16 unit N(0,1) "
                                  "(device-generated, checked against the host generator in "
                                  "tests/test_gpu_c3.py), batch sweep", "n": n, "d": d, "k": k,
                      "batches": batches, "storage": "bf16"},
           "dtype": "bf16", "steps": args.steps, "warmup": args.warmup, "batches": per_batch}

    if not args.no_cpu:
        # the oracle over the whole database, streamed to the host in chunks:
        # all cores on the sample queries, one core on query 0
        host = ctx["host"]
        th = host["threads_all_core"]
        sample = [p for p in C3_SAMPLE if p < bmax]
        xq = syn.bf16_bits_to_f32(xq16[sample])
        chunk = 1 << 20
        cd, ci, c1d, c1i = [], [], [], []
        t_all = t_one = 0.0
        for r0 in range(0, n, chunk):
            rows = idx.reconstruct_n(r0, min(chunk, n - r0))
            t = time.perf_counter()
            Dc, Ic = oracle.flat_search(rows, xq, k, oracle.IP, th)
            t_all += time.perf_counter() - t
            cd.append(Dc)
            ci.append(np.where(Ic >= 0, Ic + r0, -1))
            if not args.no_single_core:
                t = time.perf_counter()
                oracle.flat_search(rows, xq[:1], k, oracle.IP, 1)
                t_one += time.perf_counter() - t
            del rows
        cd, ci = np.concatenate(cd, 1), np.concatenate(ci, 1)
        Dr = np.empty((len(sample), k), np.float32)
        Ir = np.empty((len(sample), k), np.int32)
        for j in range(len(sample)):
            o = np.lexsort((ci[j], -cd[j].astype(np.float64)))[:k]
            Dr[j], Ir[j] = cd[j][o], ci[j][o]
        where = {p: j for j, p in enumerate(sample)}
        for B in batches:
            D, I, pos = results[B]
            rows_r = [where[p] for p in pos]
            bad = knn_failures(D, I, Dr[rows_r], Ir[rows_r], 1, rtol=1e-3)
            per_batch[str(B)]["parity"] = {
                "ok": not bad, "checked_queries": len(pos), "failures": len(bad),
                "rule": "tie-aware top-k vs the oracle over all rows (bf16 values fed to both; "
                        "rel 1e-3 ties)", "positions": pos}
        one = (1 / t_one, 1, t_one) if not args.no_single_core else None
        out["cpu_baseline"] = cpu_baseline_entry(
            (len(sample) / t_all, len(sample), t_all), one, "queries/s",
            "{n} queries against all " + f"{n} rows, streamed in 1M-row chunks" +
            " ({t:.1f} s of oracle time), fp64 oracle", host)
    qbuf.free()
    Dbuf.free()
    Ibuf.free()
    idx.close()
    return out


# --------------------------------------------------------------------------
# C4: k-means step
# --------------------------------------------------------------------------
def run_kmeans(vs, NN, args, ctx):
    """one Lloyd iteration (assign + update) per step over 2M x 256
    fp32 points from a 1,024-component mixture, 4,096 centroids from a seeded
    subset; the centroids of step i feed step i + 1 (kmeans.dart:91-140)."""
    import oracle
    from vector_store import synthetic as syn

    n, d, ncomp, K = args.n or 2_000_000, 256, 1024, 4096
    x, _ = syn.gaussian_mixture(n, d, ncomp, 0.1, args.seed)
    cen = x[syn.seeded_subset(n, K, args.seed)].copy()
    pts = vs.GpuIndexFlat.l2(d, storage="f32")
    pts.add(x)

    def jitter(step):  # the reference draws these from dart:math Random (kmeans.dart:128-138)
        return syn.rng(args.seed + 7, step).random(K * d)

    for w in range(args.warmup):
        _, cen, _, _ = vs.kmeans_step(pts, cen, 1, jitter(w))
    jits = [jitter(args.warmup + i) for i in range(args.steps)]
    # each timed step's results go to its own caller buffers, allocated and
    # touched before the clock starts (the reference's train loop also
    # reuses one assignment buffer); every step's results are kept for the
    # parity checks
    outs = []
    for _ in range(args.steps):
        o = (np.empty(n, np.int32), np.empty((K, d), np.float32), np.empty(K, np.int32))
        for arr in o:
            arr.fill(0)
        outs.append(o)
    pts.prof_enable(True)
    pts.prof_reset()
    cen_first = cen.copy()
    hist = []  # per timed step: input centroids, assignments, new centroids, objective
    times = []
    t0 = time.perf_counter()
    for i in range(args.steps):
        t = time.perf_counter()
        cin = cen
        a, cen, cnt, obj = vs.kmeans_step(pts, cen, 1, jits[i], out=outs[i])
        times.append(time.perf_counter() - t)
        hist.append((cin, a, cen, obj))
    first = hist[0][1:]
    wall = time.perf_counter() - t0
    log(f"[bench] c4: {args.steps} k-means steps in {wall:.3f} s")
    pts.prof_enable(False)
    fam = {f: pts.prof_get(f) for f in ("assign", "pick", "exhaustive", "update")}
    nsc, scan_s = kernel_avg(pts, "assign")
    passes = mfma_passes(pts)
    traffic, tsrc = MEASURED_TRAFFIC.get(("c4", n, K, d), (None, None))
    roof = roofline("mfma", 2.0 * n * K * d, scan_s, ctx["peaks"], "assign scan", nsc, traffic, tsrc,
                    peak_div=passes,
                    extra={"peak_note": f"bf16 dense MFMA peak / {passes} pass(es) per distance"})
    out = {"metric": "k-means assign+update, points per second per iteration",
           "value": round(n * args.steps / wall, 1), "unit": "points/s", "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 3),
           "steps_ms": step_stats(times), "dtype": "fp32",
           "config": {"workload": f"c4: k-means step, {n} x {d} fp32 mixture of {ncomp}, K={K}, "
                                  "host centroids in/out", "n": n, "d": d, "K": K},
           "roofline": roof,
           "families_ms": {f: round(v[1] / max(v[0], 1), 3) for f, v in fam.items()},
           "exhaustive_points_per_step": pts.prof_get("kmeans_fallback_points")[0] / args.steps}
    if not args.no_cpu:
        host = ctx["host"]
        th = host["threads_all_core"]

        def timed_assign(threads, target):
            m0 = min(n, threads * 64)
            t = time.perf_counter()
            oracle.kmeans_assign(x[:m0], cen_first, threads)
            per_point = (time.perf_counter() - t) / m0
            m = int(min(n, max(m0, target / max(per_point, 1e-9))))
            t = time.perf_counter()
            a_or, _, _ = oracle.kmeans_assign(x[:m], cen_first, threads)
            dt = time.perf_counter() - t
            return m / dt, m, dt, a_or

        qa, ma, ta, a_or = timed_assign(th, args.cpu_seconds)
        one = None
        if not args.no_single_core:
            q1, m1, t1, _ = timed_assign(1, args.cpu_seconds / 2)
            one = (q1, m1, t1)
        out["cpu_baseline"] = cpu_baseline_entry(
            (qa, ma, ta), one, "points/s (assign only)",
            "assign of the first {n} points against " + f"{K} centroids" + " ({t:.1f} s), fp64 oracle",
            host)
        # parity of the first timed step: assignments on the oracle's prefix,
        # and the whole update recomputed by the oracle from the GPU's
        # (prefix-checked) assignments
        a_gpu, cen_gpu, _ = first
        same_assign = bool(np.array_equal(a_gpu[:ma], a_or))
        cen_or, _, _ = oracle.kmeans_update(x, a_gpu, cen_first, 1, jits[0])
        same_cen = bool(np.array_equal(cen_or.view(np.uint32), cen_gpu.view(np.uint32)))
        full = kmeans_full_parity(x, hist, jits, th)
        out["parity"] = {"ok": same_assign and same_cen and full["ok"],
                         "assign_equal_on_prefix": same_assign,
                         "prefix_points": int(ma), "centroids_bit_identical": same_cen,
                         "rule": "first timed step: assignments identical to the oracle's on the "
                                 "timed prefix; new centroids bit-identical to the oracle's update",
                         "full_size": full}
    pts.close()
    return out


def kmeans_full_parity(x, hist, jits, threads, sample=32768):
    """Steps of the timed loop checked over all n points: on the first and
    the last timed step, the assignments of a stride sample spread over every
    point against the oracle's (kmeans.dart:91-105, with that step's input
    centroids), the whole update recomputed by the oracle from the GPU's
    assignments (bit-identical, kmeans.dart:107-140), and (first step) the
    objective: the fp64 distance of every point to its assigned centroid,
    summed in point order."""
    import oracle

    n = len(x)
    pts = np.arange(0, n, max(1, n // sample))
    steps = []
    for si in sorted({0, len(hist) - 1}):
        cin, a_gpu, cout, obj = hist[si]
        a_or, _, _ = oracle.kmeans_assign(x[pts], cin, threads)
        cen_or, _, _ = oracle.kmeans_update(x, a_gpu, cin, 1, jits[si])
        st = {"step": si, "sample_points": int(len(pts)),
              "assign_mismatches": int(np.count_nonzero(a_gpu[pts] != a_or)),
              "centroids_bit_identical": bool(np.array_equal(cen_or.view(np.uint32),
                                                             cout.view(np.uint32)))}
        if si == 0:
            dist = np.empty(n)
            for c in range(0, n, 1 << 16):
                diff = x[c:c + (1 << 16)].astype(np.float64) - cin[a_gpu[c:c + (1 << 16)]]
                dist[c:c + (1 << 16)] = np.cumsum(diff * diff, axis=1)[:, -1]
            st["objective_equal"] = bool(np.cumsum(dist)[-1] == obj)
        steps.append(st)
    ok = all(s["assign_mismatches"] == 0 and s["centroids_bit_identical"] and
             s.get("objective_equal", True) for s in steps)
    return {"ok": ok, "steps": steps,
            "rule": "first and last timed step: assignments of a stride sample of all points "
                    "identical to the oracle's; update bit-identical; first step's objective "
                    "equal to the fp64 point-order sum of its assignments' distances"}


# --------------------------------------------------------------------------
# C5: self-join
# --------------------------------------------------------------------------
def fp64_dots(x, i, j, chunk=1 << 15):
    """fp64 dot of rows i[t], j[t] summed in dimension order (index.dart dot)."""
    out = np.empty(len(i))
    for c in range(0, len(i), chunk):
        p = x[i[c:c + chunk]].astype(np.float64) * x[j[c:c + chunk]].astype(np.float64)
        out[c:c + chunk] = np.cumsum(p, axis=1)[:, -1]
    return out


def join_full_parity(x, pi, pj, ps, thr, planted):
    """The whole self-join output against what fixes it at full size: every
    emitted pair (i < j, sorted, unique) re-scored in fp64 is >= thr and its
    score is the fp32 of that value; every planted pair (a base vector and
    its copies, the only pairs near thr: random pairs of unit N(0,1) vectors
    at d = 512 sit about 21 sigma below) is emitted exactly when its fp64
    score is >= thr."""
    n = len(x)
    pi, pj = pi.astype(np.int64), pj.astype(np.int64)
    key = pi * n + pj
    ordered = bool(np.all(pi < pj) and np.all(np.diff(key) > 0))
    s64 = fp64_dots(x, pi, pj)
    rescored = bool(np.all(s64 >= thr))
    scores = bool(np.array_equal(ps.view(np.uint32), s64.astype(np.float32).view(np.uint32)))
    qi, qj = planted
    qs = fp64_dots(x, qi, qj)
    emitted = np.isin(qi * n + qj, key)
    wrong = int(np.count_nonzero(emitted != (qs >= thr)))
    outside = int(np.count_nonzero(~np.isin(key, qi * n + qj)))
    return {"ok": ordered and rescored and scores and wrong == 0,
            "pairs_emitted": int(len(pi)), "sorted_unique_i_lt_j": ordered,
            "emitted_rescored_ge_threshold": rescored, "scores_fp32_of_fp64": scores,
            "planted_pairs_checked": int(len(qi)),
            "planted_pairs_within_1e-3_of_threshold": int(np.count_nonzero(np.abs(qs - thr) < 1e-3)),
            "planted_pair_failures": wrong, "emitted_outside_planted": outside,
            "rule": "every emitted pair re-scored in fp64 (>= threshold, fp32 score of it); "
                    "every planted pair emitted iff its fp64 score >= threshold"}


def run_join(vs, NN, args, ctx):
    """near-duplicate cosine self-join of 500k x 512 fp32 unit
    vectors (5% planted copies), all pairs i < j with dot >= 0.95 sorted by
    (i, j) (vector_dedup_demo.dart:115-128).  One step = one self-join."""
    import oracle
    from vector_store import synthetic as syn

    n, d, thr = args.n or 500_000, 512, 0.95
    x = syn.dedup_set(n, d, 0.05, 0.01, args.seed)
    g = vs.GpuIndexFlat(d, vs.Metric(1), storage="f32")
    g.add(x)
    for _ in range(args.warmup):
        g.self_join(thr)
    g.prof_enable(True)
    g.prof_reset()
    res = {}

    def step():
        res["p"] = g.self_join(thr)

    wall, times = time_steps(step, args.steps, 0, "c5 self-join")
    g.prof_enable(False)
    pi, pj, ps = res["p"]
    nj, join_s = kernel_avg(g, "join")
    passes = mfma_passes(g)
    traffic, tsrc = MEASURED_TRAFFIC.get(("c5", n, n, d), (None, None))
    roof = roofline("mfma", 2.0 * d * n * (n - 1) / 2, join_s, ctx["peaks"],
                    "join scan (upper triangle)", nj, traffic, tsrc, peak_div=passes,
                    extra={"peak_note": f"bf16 dense MFMA peak / {passes} pass(es) per distance",
                           "refine_avg_ms": round(kernel_avg(g, "refine")[1] * 1e3, 3)})
    out = {"metric": "cosine self-join, vectors per second", "value": round(n * args.steps / wall, 1),
           "unit": "vectors/s", "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(wall / args.steps * 1e3, 3), "steps_ms": step_stats(times),
           "dtype": "fp32",
           "config": {"workload": f"c5: self-join {n} x {d} fp32 unit, 5% planted duplicates, "
                                  f"cos >= {thr}", "n": n, "d": d, "pairs": int(len(pi))},
           "roofline": roof}
    if not args.no_cpu:
        host = ctx["host"]

        def timed_rows(threads, target):
            t = time.perf_counter()
            oracle.self_join(x, thr, row_begin=0, row_end=threads, nthreads=threads)
            per_row = (time.perf_counter() - t) / threads
            rows = int(max(threads, target / max(per_row, 1e-9)))
            rows = min(rows, n)
            t = time.perf_counter()
            ri, rj, _ = oracle.self_join(x, thr, row_begin=0, row_end=rows, nthreads=threads)
            dt = time.perf_counter() - t
            work = sum(n - 1 - i for i in range(rows))
            total = n * (n - 1) / 2
            return n / (dt * total / work), rows, dt, (ri, rj)

        th = host["threads_all_core"]
        qa, ra, ta, (ri, rj) = timed_rows(th, args.cpu_seconds)
        one = None
        if not args.no_single_core:
            q1, r1, t1, _ = timed_rows(1, args.cpu_seconds / 2)
            one = (q1, r1, t1)
        out["cpu_baseline"] = cpu_baseline_entry(
            (qa, ra, ta), one, "vectors/s",
            "rows 0..{n} of the upper triangle ({t:.1f} s), extrapolated linearly to all " +
            f"{n} rows; fp64 oracle", host)
        sel = pi < ra
        agree = bool(np.array_equal(ri, pi[sel]) and np.array_equal(rj, pj[sel]))
        full = join_full_parity(x, pi, pj, ps, thr, syn.dedup_planted_pairs(n, 0.05, args.seed))
        out["parity"] = {"ok": agree and full["ok"], "rows_checked": int(ra),
                         "pairs_checked": int(len(ri)),
                         "rule": "pair list (i, j) identical to the oracle's for every i in the "
                                 "checked rows", "full_size": full}
    g.close()
    return out


# --------------------------------------------------------------------------
# yardsticks
# --------------------------------------------------------------------------
def run_copy_calibration(args):
    """A plain device copy of known size (the library's copy16 kernel), the
    yardstick for the FETCH_SIZE / WRITE_SIZE counters: under rocprofv3 --pmc
    its per-dispatch KiB, divided by the bytes it must move, is the scale
    factor applied to the scan kernel's counter readings."""
    from vector_store import _native as NN

    nbytes = args.n or 1 << 30
    src, dst = NN.DeviceBuffer(nbytes), NN.DeviceBuffer(nbytes)
    lib = NN.load()
    for _ in range(args.warmup):
        NN.check(lib.vs_dev_copy(0, dst.ptr, src.ptr, nbytes))
    t = time.perf_counter()
    for _ in range(args.steps):
        NN.check(lib.vs_dev_copy(0, dst.ptr, src.ptr, nbytes))
    dt = (time.perf_counter() - t) / args.steps
    src.free()
    dst.free()
    return {"workload": "copy", "bytes_read": nbytes, "bytes_written": nbytes,
            "ms": round(dt * 1e3, 4), "GBps_read_plus_write": round(2 * nbytes / dt / 1e9, 1)}


def run_library_gemm(args):
    """For scale only (not the product path): the vendor library's bf16 GEMM
    through torch (hipBLASLt on ROCm) on the K = 768 shapes of configs[2] at
    batch 1024 and 8192, output written in bf16, no selection."""
    import torch

    rows = []
    for m, n in ((1024, 262_144), (1024, 1_048_576), (8192, 65_536)):
        a = torch.randn(m, 768, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(n, 768, device="cuda", dtype=torch.bfloat16)
        for _ in range(max(args.warmup, 1)):
            c = a @ b.t()
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(args.steps):
            c = a @ b.t()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t) / args.steps
        rows.append({"m": m, "n": n, "k": 768, "ms": round(dt * 1e3, 3),
                     "tflops": round(2 * m * n * 768 / dt / 1e12, 1)})
        del a, b, c
    return {"workload": "libgemm", "note": "library bf16 GEMM for scale, not the product path",
            "shapes": rows}


def guarded(name, fn):
    try:
        return fn()
    except Exception as e:  # one failing workload must not hide the others
        log(f"[bench] {name} failed: {type(e).__name__}: {e}")
        return {"error": f"{type(e).__name__}: {e}"[:500]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="all",
                    choices=["all", "c1", "c2", "c2f", "c3", "c4", "c5", "copy", "libgemm"])
    ap.add_argument("--batch", type=int, default=0, help="c3 alone: one batch size")
    ap.add_argument("--c3-batches", default="1,64,1024,8192")
    ap.add_argument("--n", type=int, default=0)
    ap.add_argument("--nq", type=int, default=0)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--k", type=int, default=0, help="override the workload's k")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-single-core", action="store_true")
    ap.add_argument("--csv", default="", help="write the benchIndex rows as CSV (toBenchCsv)")
    ap.add_argument("--md", default="", help="write the benchIndex rows as Markdown")
    ap.add_argument("--opt", action="append", default=[], metavar="NAME=VALUE",
                    help="planner option set on every index (vs_index_set_option), for "
                         "profiling runs of a kernel variant; the default run sets none")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding of this path is a design note, not built.", file=sys.stderr)
        sys.exit(2)
    if args.workload == "libgemm":  # torch only; the library is not loaded
        print(json.dumps(run_library_gemm(args)), flush=True)
        return
    import vector_store as vs
    from vector_store import _native as NN
    from vector_store import gpu_index_flat

    for o in args.opt:
        name, _, value = o.partition("=")
        gpu_index_flat.DEFAULT_OPTIONS[name] = int(value)
    if vs.device_count() < 1:
        raise SystemExit("no HIP device visible")
    if args.workload == "copy":
        print(json.dumps(run_copy_calibration(args)), flush=True)
        return
    ctx = {"host": host_info(), "peaks": measured_peaks(NN)}
    log(f"[bench] host {ctx['host']}, measured peaks {ctx['peaks']}")
    if args.workload == "all":
        out = run_search(vs, NN, "c2", args, ctx, full=True)
        batches = [int(b) for b in args.c3_batches.split(",") if b]
        args_n = args.n
        args.n = 0  # --n applies to single workloads only
        out["workloads"] = {
            "c1": guarded("c1", lambda: run_search(vs, NN, "c1", args, ctx)),
            "c2f": guarded("c2f", lambda: run_search(vs, NN, "c2f", args, ctx)),
            "c3": guarded("c3", lambda: run_c3(vs, NN, args, ctx, batches)),
            "c4": guarded("c4", lambda: run_kmeans(vs, NN, args, ctx)),
            "c5": guarded("c5", lambda: run_join(vs, NN, args, ctx)),
        }
        args.n = args_n
        oks = [out.get("parity", {}).get("ok")]
        for w, r in out["workloads"].items():
            if w == "c3" and "batches" in r:
                oks += [b.get("parity", {}).get("ok") for b in r["batches"].values()]
            else:
                oks.append(r.get("parity", {}).get("ok"))
        out["parity_all_ok"] = all(o is True for o in oks) if not args.no_cpu else None
    elif args.workload in ("c1", "c2", "c2f"):
        out = run_search(vs, NN, args.workload, args, ctx, full=True)
    elif args.workload == "c3":
        batches = [args.batch] if args.batch else [int(b) for b in args.c3_batches.split(",") if b]
        out = run_c3(vs, NN, args, ctx, batches)
    elif args.workload == "c4":
        out = run_kmeans(vs, NN, args, ctx)
    else:
        out = run_join(vs, NN, args, ctx)
    out["host"] = ctx["host"]
    out["measured_peaks"] = ctx["peaks"]
    if args.opt:
        out["options"] = dict(gpu_index_flat.DEFAULT_OPTIONS)
    if ctx.get("bench_rows"):
        from vector_store.bench import to_bench_csv, to_bench_markdown

        if args.csv:
            open(args.csv, "w").write(to_bench_csv(ctx["bench_rows"]))
        if args.md:
            open(args.md, "w").write(to_bench_markdown(ctx["bench_rows"]))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
