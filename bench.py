"""Benchmark of the MI355X flat k-NN path (one JSON line on stdout).

Default workload = BASELINE.json configs[1]: exact L2 top-100 over a
1,000,000 x 128 database of integers 0..255 stored as fp32, 10,000 queries of
the same distribution.  One step = one search of the whole query batch with
the database, the queries and the result buffers resident in HBM.

value = queries per second over the K timed steps.  roofline = the scan
kernel (the dominant launch) timed with HIP events on the index's stream:
algorithmic flops per launch (2 * nq * N * d) over its mean duration, against
the peak of the MFMA instruction it runs (bf16 for lossless-bf16 storage).
cpu_baseline = the CPU oracle (a restatement of IndexFlat.search,
index_flat.dart:62-97) on this host's cores over a bounded query sample of
the same database, scaled to queries per second.

Other workloads (--workload c1|c3|c4|c5) exist for exploration and profiling.
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

# HBM bytes per launch of the dominant kernel, measured with two rocprofv3
# --pmc runs (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0: the factors a plain 16-byte
# copy of known size reads, profiles/copy16_calibration.md), keyed by
# (workload, n, nq, k).  The command and readings are in the named profile;
# configurations without a measurement report traffic null.
MEASURED_TRAFFIC = {
    ("c2", 1_000_000, 10_000, 100): (1.09e9, "profiles/scan_c2_1Mx128_k100.md"),
    ("c3", 20_000_000, 1, 10): (30.88e9, "profiles/scan_c3_20Mx768_b1_b64.md"),
}


def mfma_passes(idx):
    """bf16 MFMA passes per distance of an fp32-row scan: 1 when the one-pass
    bf16 selection ran (GEMM shapes of storage code 2, or 1 on the bf16 copy
    of the rows, or the row-shared scan, which reads fp32 rows only that
    way), else 3 (hi*q0 + lo*q0 + hi*q1 of the split-bf16 planes)."""
    coarse = sum(idx.prof_get(f"gemm:{st},1,2,{wq},4,2,32")[0] for st in (1, 2) for wq in (2, 4))
    coarse += idx.prof_get("shared")[0]
    return 1 if coarse else 3


def measured_traffic(workload, n, nq, k):
    hit = MEASURED_TRAFFIC.get((workload, n, nq, k))
    return (hit[0], hit[1]) if hit else (None, None)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def host_info():
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    return cpu, cores


def cpu_baseline(xb, xq, k, metric, target_s, threads):
    """Times the oracle on a bounded sample of the batch; returns (qps, sample, results)."""
    import oracle

    n0 = min(len(xq), max(threads, 4))
    t = time.perf_counter()
    oracle.flat_search(xb, xq[:n0], k, metric, threads)
    per_q = (time.perf_counter() - t) / n0
    ns = int(min(len(xq), max(n0, target_s / max(per_q, 1e-9))))
    ns = max(threads, (ns // threads) * threads) if ns >= threads else ns
    t = time.perf_counter()
    D, I = oracle.flat_search(xb, xq[:ns], k, metric, threads)
    dt = time.perf_counter() - t
    return ns / dt, ns, dt, (D, I)


def run_search_workload(args, vs, syn, N):
    from vector_store import _native as NN

    if args.workload == "c2":
        n, d, nq, k, metric = args.n or 1_000_000, 128, args.nq or 10_000, args.k or 100, 0
        xb = syn.int_grid(n, d, args.seed, 0)
        xq = syn.int_grid(nq, d, args.seed, 1)
        storage, qdt = "auto", NN.VS_DTYPE_F32
        desc = f"c2: exact L2 top-{k}, {n} x {d} fp32 integers 0..255, {nq} queries"
    elif args.workload == "c1":
        n, d, nq, k, metric = args.n or 10_000, 384, args.nq or 100, args.k or 10, 1
        xb = syn.normal_unit(n, d, args.seed, 0)
        xq = syn.normal_unit(nq, d, args.seed, 1)
        storage, qdt = "f32", NN.VS_DTYPE_F32
        desc = f"c1: exact IP top-{k}, {n} x {d} fp32 unit N(0,1), {nq} queries"
    elif args.workload == "c3":
        n, d, nq, k, metric = args.n or 20_000_000, 768, args.nq or args.batch, args.k or 10, 1
        xb = None
        xq = syn.to_bf16_bits(syn.normal_unit(nq, d, args.seed, 1))
        storage, qdt = "bf16", NN.VS_DTYPE_BF16
        desc = f"c3: exact IP top-{k}, {n} x {d} bf16 unit N(0,1) (device-generated), batch {nq}"
    else:
        raise SystemExit(f"unknown search workload {args.workload}")

    idx = vs.GpuIndexFlat(d, vs.Metric(metric), storage=storage)
    t0 = time.perf_counter()
    if xb is not None:
        idx.add(xb)
    else:
        idx.reserve(n)
        chunk = 1 << 20
        buf = NN.DeviceBuffer(chunk * d * 2)
        for r in range(0, n, chunk):
            m = min(chunk, n - r)
            NN.check(NN.load().vs_gen_normal(0, buf.ptr, NN.VS_DTYPE_BF16, m, d, args.seed,
                                             (1 << 32) + r, 1))
            idx.add_device(buf, m, NN.VS_DTYPE_BF16)
        buf.free()
    log(f"[bench] {desc}: add {time.perf_counter() - t0:.1f}s, storage={idx.storage}")

    esz = 2 if qdt == NN.VS_DTYPE_BF16 else 4
    qbuf = NN.DeviceBuffer(nq * d * esz)
    qbuf.upload(xq)
    Dbuf = NN.DeviceBuffer(nq * k * 4)
    Ibuf = NN.DeviceBuffer(nq * k * 4)

    for _ in range(args.warmup):
        idx.search_device(qbuf, nq, k, Dbuf, Ibuf, qdt)
    idx.prof_enable(True)
    idx.prof_reset()
    t = time.perf_counter()
    for i in range(args.steps):
        idx.search_device(qbuf, nq, k, Dbuf, Ibuf, qdt)
        log(f"[bench] step {i + 1}/{args.steps} done")
    wall = time.perf_counter() - t
    idx.prof_enable(False)
    nscan, scan_ms = idx.prof_get("scan")
    nmerge, merge_ms = idx.prof_get("merge")
    npre, pre_ms = idx.prof_get("prepass")

    D = np.empty((nq, k), np.float32)
    I = np.empty((nq, k), np.int32)
    Dbuf.download(D)
    Ibuf.download(I)

    flops = 2.0 * nq * n * d
    scan_avg_s = scan_ms / max(nscan, 1) / 1e3
    bf16 = idx.storage == "bf16"
    peak = PEAK["bf16_mfma_tflops"] / (1 if bf16 else 3)  # fp32 rows: three split-bf16 passes
    achieved = flops / scan_avg_s / 1e12
    roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": measured_traffic(args.workload, n, nq, k)[0],
            "traffic_source": measured_traffic(args.workload, n, nq, k)[1],
            "kernel": "scan", "scan_kinds": {f: idx.prof_get(f)[0] for f in ("shared", "gemm", "tiled", "streamed") if idx.prof_get(f)[0]},
            "launches": nscan, "avg_ms": round(scan_avg_s * 1e3, 4),
            "algorithmic_flops_per_launch": flops, "merge_avg_ms": round(merge_ms / max(nmerge, 1), 4),
            "prepass_ms_per_step": round(pre_ms / args.steps, 4) if npre else None}
    if nq <= 64:  # streaming regime: the database bytes bound the kernel
        db_bytes = n * d * (2 if bf16 else 4)
        gbs = db_bytes / scan_avg_s / 1e9
        roof.update({"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK["hbm_gbs"],
                     "unit": "GB/s", "frac": round(gbs / PEAK["hbm_gbs"], 4),
                     "algorithmic_bytes_per_launch": db_bytes})

    out = {"metric": METRIC, "value": round(nq * args.steps / wall, 1), "unit": "queries/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None,
           "dtype": "bf16" if bf16 else "fp32", "data": "synthetic",
           "config": {"workload": desc, "n": n, "d": d, "nq": nq, "k": k,
                      "metric": "L2" if metric == 0 else "IP", "storage": idx.storage},
           "roofline": roof}

    if not args.no_cpu and xb is not None:
        cpu, cores = host_info()
        threads = min(cores, 16)
        qps, ns, dt, (Dc, Ic) = cpu_baseline(xb, xq, k, metric, args.cpu_seconds, threads)
        rec = float(np.mean([len(set(I[i]) & set(Ic[i])) / k for i in range(ns)]))
        out["cpu_baseline"] = {"value": round(qps, 3), "unit": "queries/s", "cores": threads,
                               "kind": "port",
                               "sample": f"first {ns} of the {nq} queries against the full "
                                         f"{n}-row database ({dt:.1f} s), fp64 oracle",
                               "cpu": cpu}
        out["recall_vs_cpu_sample"] = round(rec, 6)
    idx.close()
    return out


def run_kmeans_workload(args, vs, syn):
    """one Lloyd iteration (assign + update) per step over 2M x 256
    fp32 points from a 1,024-component mixture, 4,096 centroids from a seeded
    subset; the centroids of step i feed step i + 1 (kmeans.dart:91-140)."""
    import oracle

    n, d, ncomp, K = args.n or 2_000_000, 256, 1024, 4096
    x, _ = syn.gaussian_mixture(n, d, ncomp, 0.1, args.seed)
    cen = x[syn.seeded_subset(n, K, args.seed)].copy()
    pts = vs.GpuIndexFlat.l2(d, storage="f32")
    pts.add(x)
    # jitter draws for empty clusters (the reference takes them from dart:math
    # Random, kmeans.dart:128-138): seeded uniforms, one stream per step
    def jitter(step):
        return syn.rng(args.seed + 7, step).random(K * d)

    for w in range(args.warmup):
        _, cen, _, _ = vs.kmeans_step(pts, cen, 1, jitter(w))
    # the draws are inputs: made before the timed steps
    jits = [jitter(args.warmup + i) for i in range(args.steps)]
    pts.prof_enable(True)
    pts.prof_reset()
    cen0 = cen.copy()
    t = time.perf_counter()
    for i in range(args.steps):
        _, cen, _, obj = vs.kmeans_step(pts, cen, 1, jits[i])
        log(f"[bench] k-means step {i + 1}/{args.steps}: objective {obj:.6g}")
    wall = time.perf_counter() - t
    pts.prof_enable(False)
    fam = {f: pts.prof_get(f) for f in ("assign", "pick", "exhaustive", "update")}
    nfb = pts.prof_get("kmeans_fallback_points")[0]
    nsc, scan_ms = fam["assign"]
    scan_s = scan_ms / max(nsc, 1) / 1e3
    flops = 2.0 * n * K * d
    passes = mfma_passes(pts)
    achieved = flops / scan_s / 1e12
    peak = PEAK["bf16_mfma_tflops"] / passes
    out = {"metric": "k-means assign+update, points per second per iteration",
           "value": round(n * args.steps / wall, 1), "unit": "points/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": {"workload": f"c4: k-means step, {n} x {d} fp32 mixture of {ncomp}, "
                                  f"K={K}, host centroids in/out", "n": n, "d": d, "K": K},
           "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": round(peak, 1),
                        "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": None,
                        "kernel": "assign scan", "avg_ms": round(scan_s * 1e3, 3),
                        "algorithmic_flops_per_launch": flops,
                        "peak_note": f"bf16 dense MFMA peak / {passes} pass(es) per distance"},
           "families_ms": {f: round(v[1] / max(v[0], 1), 3) for f, v in fam.items()},
           "exhaustive_points_per_step": nfb / args.steps}
    if not args.no_cpu:
        cpu, cores = host_info()
        threads = min(cores, 16)
        m0 = min(n, threads * 64)
        t = time.perf_counter()
        oracle.kmeans_assign(x[:m0], cen0, threads)
        per_point = (time.perf_counter() - t) / m0
        for _ in range(3):  # re-aim while the sample runs under half the target time
            m = int(min(n, max(m0, args.cpu_seconds / max(per_point, 1e-9))))
            t = time.perf_counter()
            oracle.kmeans_assign(x[:m], cen0, threads)
            dt = time.perf_counter() - t
            per_point = dt / m
            if dt >= 0.5 * args.cpu_seconds or m == n:
                break
        out["cpu_baseline"] = {"value": round(m / dt, 1), "unit": "points/s (assign only)",
                               "cores": threads, "kind": "port",
                               "sample": f"assign of the first {m} points against {K} centroids "
                                         f"({dt:.1f} s), fp64 oracle", "cpu": cpu}
    pts.close()
    return out


def run_join_workload(args, vs, syn):
    """near-duplicate cosine self-join of 500k x 512 fp32 unit
    vectors (5% planted copies), all pairs i < j with dot >= 0.95 sorted by
    (i, j) (vector_dedup_demo.dart:115-128).  One step = one self-join."""
    import oracle

    n, d, thr = args.n or 500_000, 512, 0.95
    x = syn.dedup_set(n, d, 0.05, 0.01, args.seed)
    g = vs.GpuIndexFlat(d, vs.Metric(1), storage="f32")
    g.add(x)
    for _ in range(args.warmup):
        g.self_join(thr)
    g.prof_enable(True)
    g.prof_reset()
    t = time.perf_counter()
    for i in range(args.steps):
        pi, pj, ps = g.self_join(thr)
        log(f"[bench] self-join {i + 1}/{args.steps}: {len(pi)} pairs")
    wall = time.perf_counter() - t
    g.prof_enable(False)
    nj, join_ms = g.prof_get("join")
    join_s = join_ms / max(nj, 1) / 1e3
    flops = 2.0 * d * n * (n - 1) / 2
    passes = mfma_passes(g)
    achieved = flops / join_s / 1e12
    peak = PEAK["bf16_mfma_tflops"] / passes
    out = {"metric": "cosine self-join, vectors per second", "value": round(n * args.steps / wall, 1),
           "unit": "vectors/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(wall / args.steps * 1e3, 3), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": {"workload": f"c5: self-join {n} x {d} fp32 unit, 5% planted duplicates, "
                                  f"cos >= {thr}", "n": n, "d": d, "pairs": int(len(pi))},
           "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": round(peak, 1),
                        "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": None,
                        "kernel": "join scan (upper triangle)", "avg_ms": round(join_s * 1e3, 3),
                        "algorithmic_flops_per_launch": flops,
                        "peak_note": f"bf16 dense MFMA peak / {passes} pass(es) per distance"}}
    if not args.no_cpu:
        cpu, cores = host_info()
        threads = min(cores, 16)
        t = time.perf_counter()
        oracle.self_join(x, thr, row_begin=0, row_end=threads, nthreads=threads)
        per_row = (time.perf_counter() - t) / threads
        rows = int(max(threads, args.cpu_seconds / max(per_row, 1e-9)))
        t = time.perf_counter()
        ri, rj, _ = oracle.self_join(x, thr, row_begin=0, row_end=rows, nthreads=threads)
        dt = time.perf_counter() - t
        work = sum(n - 1 - i for i in range(rows))
        total = n * (n - 1) / 2
        agree = bool(np.array_equal(ri, pi[pi < rows]) and np.array_equal(rj, pj[pi < rows]))
        out["cpu_baseline"] = {"value": round(n / (dt * total / work), 3), "unit": "vectors/s",
                               "cores": threads, "kind": "port",
                               "sample": f"rows 0..{rows - 1} of the upper triangle ({dt:.1f} s), "
                                         f"extrapolated linearly to all {n} rows; fp64 oracle",
                               "cpu": cpu}
        out["pairs_match_cpu_sample"] = agree
    g.close()
    return out


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c2")
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--n", type=int, default=0)
    ap.add_argument("--nq", type=int, default=0)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--k", type=int, default=0, help="override the workload's k")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "sharding of this path is a design note, not built.", file=sys.stderr)
        sys.exit(2)
    if args.workload == "libgemm":  # torch only; the library is not loaded
        print(json.dumps(run_library_gemm(args)), flush=True)
        return
    import vector_store as vs
    from vector_store import synthetic as syn

    if vs.device_count() < 1:
        raise SystemExit("no HIP device visible")
    if args.workload == "copy":
        out = run_copy_calibration(args)
    elif args.workload == "c4":
        out = run_kmeans_workload(args, vs, syn)
    elif args.workload == "c5":
        out = run_join_workload(args, vs, syn)
    else:
        out = run_search_workload(args, vs, syn, None)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
