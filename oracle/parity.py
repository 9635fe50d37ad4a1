"""Parity comparison of GPU results with the CPU oracle's.

TEST INFRASTRUCTURE ONLY (used by tests/ and by bench.py's parity fields).

Distances: the GPU re-ranks its survivors with the reference's exact fp64
arithmetic, so a neighbour present on both sides must carry a bit-identical
fp32 distance.  Ids: identical except inside tie groups -- neighbours whose
oracle distances lie within `rtol` (+ `atol`) of each other (BASELINE
north_star: rel 1e-5 for fp32 data, 1e-3 for bf16 data fed identically to
both sides).
"""
import numpy as np


def _close(a, b, rtol, atol):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    with np.errstate(invalid="ignore"):
        both_inf = np.isinf(a) & np.isinf(b) & (np.sign(a) == np.sign(b))
        return both_inf | (np.abs(a - b) <= atol + rtol * np.maximum(np.abs(a), np.abs(b)))


def knn_failures(D, I, Dr, Ir, metric, rtol=1e-5, atol=1e-6, exact_shared=True, xb=None,
                 xq=None):
    """Queries whose (D, I) differ from the oracle's (Dr, Ir) beyond ties.

    metric 0 = L2 (ascending), 1 = IP (descending).  The last tie group --
    oracle distances tied with the k-th -- may continue past k, so the ids
    there may differ (the reference keeps whichever tied rows its heap
    history left, index.dart:248-260).  Given xb and xq, every GPU id the
    oracle does not list is checked to lie at its reported distance
    (recomputed in fp64).  Returns a list of (query, reason, ...) tuples."""
    D, I, Dr, Ir = map(np.asarray, (D, I, Dr, Ir))
    if D.shape != Dr.shape or I.shape != Ir.shape:
        return [(-1, "shape", D.shape, Dr.shape)]
    nq, k = Dr.shape
    bad = []
    for q in range(nq):
        if not _close(D[q], Dr[q], rtol, atol).all():
            bad.append((q, "distances", D[q][:5], Dr[q][:5]))
            continue
        if not np.array_equal(Ir[q] < 0, I[q] < 0):  # sentinel positions agree exactly
            bad.append((q, "sentinels", I[q], Ir[q]))
            continue
        valid = Ir[q] >= 0
        if not valid.any():
            continue
        kth = Dr[q][valid][-1]
        sgn = 1.0 if metric == 0 else -1.0
        # oracle neighbours clearly better than the k-th must all be found
        tol = atol + rtol * abs(kth)
        clear = valid & (sgn * (kth - Dr[q]) > tol)
        missing = set(Ir[q][clear].tolist()) - set(I[q].tolist())
        if missing:
            bad.append((q, "missing", sorted(missing)[:5]))
            continue
        # position-wise ids where the oracle distance is not tied with a neighbour
        for j in np.nonzero(valid)[0]:
            lo = Dr[q][j - 1] if j > 0 else None
            hi = Dr[q][j + 1] if j + 1 < k and Ir[q][j + 1] >= 0 else None
            tied = (lo is not None and _close(lo, Dr[q][j], rtol, atol)) or (
                hi is not None and _close(hi, Dr[q][j], rtol, atol)) or (
                _close(kth, Dr[q][j], rtol, atol))
            if not tied and I[q][j] != Ir[q][j]:
                bad.append((q, "id", j, I[q][j], Ir[q][j]))
                break
        if xb is not None:
            known = set(Ir[q].tolist())
            for i, d in zip(I[q], D[q]):
                if int(i) >= 0 and int(i) not in known:
                    x = np.asarray(xb[int(i)], np.float64)
                    y = np.asarray(xq[q], np.float64)
                    true = float(np.sum((x - y) ** 2)) if metric == 0 else float(np.dot(x, y))
                    if not _close(true, d, rtol, atol):
                        bad.append((q, "wrong distance for extra id", int(i), float(d), true))
                        break
        if exact_shared:
            ref = {int(i): float(d) for i, d in zip(Ir[q], Dr[q]) if i >= 0}
            for i, d in zip(I[q], D[q]):
                if int(i) in ref and np.float32(d) != np.float32(ref[int(i)]):
                    bad.append((q, "not bit-exact", int(i), float(d), ref[int(i)]))
                    break
    return bad


def range_equal(lims, D, I, lims_r, Dr, Ir):
    """Range results identical: CSR limits, ids ascending per query, fp32
    distances bit for bit."""
    return (np.array_equal(np.asarray(lims, np.int64), np.asarray(lims_r, np.int64))
            and np.array_equal(I, Ir)
            and np.array_equal(np.asarray(D, np.float32).view(np.uint32),
                               np.asarray(Dr, np.float32).view(np.uint32)))
