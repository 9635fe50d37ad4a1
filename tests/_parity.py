"""Parity assertions between the GPU results and the CPU oracle (the
comparison itself lives in oracle/parity.py, shared with bench.py)."""
import numpy as np

from oracle.parity import knn_failures, range_equal


def assert_knn_parity(D, I, Dr, Ir, metric, rtol=1e-5, atol=1e-6, exact_shared=True,
                      xb=None, xq=None):
    """metric 0 = L2 (ascending), 1 = IP (descending); ids equal except in
    tie groups, shared neighbours' distances bit-identical."""
    bad = knn_failures(D, I, Dr, Ir, metric, rtol, atol, exact_shared, xb, xq)
    assert not bad, f"{len(bad)} queries differ; first: {bad[:3]}"


def assert_range_parity(lims, D, I, lims_r, Dr, Ir):
    """Range results: identical CSR (ids ascending per query, fp32 of the fp64 score)."""
    assert np.array_equal(np.asarray(lims, np.int64), np.asarray(lims_r, np.int64)), "limits differ"
    assert np.array_equal(I, Ir), "ids differ"
    assert range_equal(lims, D, I, lims_r, Dr, Ir), "distances not bit-identical"
