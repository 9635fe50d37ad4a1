"""Writes tests/golden/flat_fixtures.json: expected top-5 inner-product
neighbours of the reference's two FAISDART IndexFlatIP fixtures
(data/docs_index/index.bin, data/qa_index/index.bin, copied here as
docs_index.bin / qa_index.bin), every stored vector used as a query.

Expected values come from numpy's fp64 matrix product (BLAS order), an
evaluator independent of the oracle's sequential loop; scores are rounded
to fp32 and kept with their fp64 value so tests can allow the last-bit
difference two summation orders may produce.  Run from the repo root:
    python tests/golden/make_golden.py
"""
import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def read(name):
    b = open(os.path.join(HERE, name), "rb").read()
    d, metric, n, _ = struct.unpack_from("<IIIB", b, 16)
    return metric, np.frombuffer(b, "<f4", n * d, 29).reshape(n, d)


out = {}
for name in ("docs_index.bin", "qa_index.bin"):
    metric, x = read(name)
    s = x.astype(np.float64) @ x.astype(np.float64).T
    order = np.argsort(-s, axis=1, kind="stable")[:, :5]
    off = s - np.diag(np.full(len(x), np.inf))
    out[name] = {
        "metric": int(metric),
        "top5_ids": order.tolist(),
        "top5_scores_f64": np.take_along_axis(s, order, 1).tolist(),
        "max_offdiag": float(off.max()),
    }
with open(os.path.join(HERE, "flat_fixtures.json"), "w") as f:
    json.dump(out, f, indent=1)
print("wrote flat_fixtures.json", {k: round(v["max_offdiag"], 4) for k, v in out.items()})
