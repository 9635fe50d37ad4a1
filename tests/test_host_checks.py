"""CPU checks of host-side pieces the GPU tests and the bench rely on:
the host restatement of the device generator (Philox4x32-10 known-answer
vectors of Random123, Salmon et al. SC'11; Box-Muller closed forms;
L2NormTransform order), and recall@k as bench.dart:356-371 defines it."""
import numpy as np

from _philox import normalized_rows, philox4x32_10, raw_rows
from vector_store import SearchResult, recall_at_k


def test_philox_known_answers():
    kat = [((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
           ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF),
            (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
           ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
            (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1))]
    for ctr, key, want in kat:
        got = philox4x32_10(np.array([ctr], np.uint32), key)[0]
        assert [int(v) for v in got] == list(want)


def test_normals_moments_and_normalisation():
    z = raw_rows(np.arange(64), 1024, 1234, 1 << 32)
    assert abs(float(z.mean())) < 0.01 and abs(float(z.var()) - 1.0) < 0.02
    x = normalized_rows(np.arange(8), 768, 1234, 7)
    n2 = (x.astype(np.float64) ** 2).sum(1)
    assert np.all(np.abs(n2 - 1.0) < 1e-6)
    # the fp64 sum runs in dimension order: its result, not a pairwise sum's,
    # sets inv (the two differ in the last bits for some rows)
    zz = raw_rows([3], 768, 1234, 7)[0].astype(np.float64)
    s = 0.0
    for v in zz:
        s = s + v * v
    want = (zz * (1.0 / np.sqrt(s))).astype(np.float32)
    assert np.array_equal(normalized_rows([3], 768, 1234, 7)[0], want)


def test_recall_at_k_rules():
    """|result ∩ truth| / (nq k); truth ids of -1 are not gold; result -1 never hits."""
    truth = SearchResult(np.zeros((2, 3), np.float32), np.array([[1, 2, -1], [4, 5, 6]], np.int32))
    res = SearchResult(np.zeros((2, 3), np.float32), np.array([[2, -1, 9], [6, 5, 4]], np.int32))
    assert recall_at_k(res, truth, 3) == (1 + 3) / 6
    empty = SearchResult(np.zeros((0, 3), np.float32), np.zeros((0, 3), np.int32))
    assert recall_at_k(empty, empty, 3) == 0.0
    # only the first k columns of either side count: gold {1, 2} / {4, 5}
    assert recall_at_k(res, truth, 2) == (1 + 1) / 4
    assert recall_at_k(res, truth, 1) == 0.0
