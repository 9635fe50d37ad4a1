"""Flat index files loaded through the C ABI (vs_index_load_flat /
vs_index_load_flat_buffer) straight into HBM: the reference's own FAISDART
fixtures (data/*/index.bin, index_io.dart:8-26, index_flat.dart:165-188) and
FAISS IndexFlat blobs (faiss_io.dart:1501-1522, 1690-1716), including the
53-byte IxF2 golden of vector_store_test.dart:1018-1093.  Searches on the
loaded index match the oracle on the host-parsed vectors."""
import os

import numpy as np
import pytest

import oracle
from _parity import assert_knn_parity
from vector_store import io as vio

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = bytes([0x49, 0x78, 0x46, 0x32, 0x02, 0, 0, 0, 0x01, 0, 0, 0, 0, 0, 0, 0,
                0, 0, 0x10, 0, 0, 0, 0, 0, 0, 0, 0x10, 0, 0, 0, 0, 0, 0x01,
                0x01, 0, 0, 0, 0x08, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0x40, 0x40, 0, 0, 0x80, 0x40])


@pytest.mark.parametrize("name", ["docs_index.bin", "qa_index.bin"])
@pytest.mark.parametrize("via", ["path", "buffer"])
def test_faisdart_fixtures(vs, name, via):
    path = os.path.join(HERE, "golden", name)
    hdr, x = vio.read_faisdart_flat(path)
    g = vs.GpuIndexFlat.load(path if via == "path" else open(path, "rb").read(), storage="f32")
    assert (g.d, int(g.metric), g.ntotal, g.is_trained) == (hdr["d"], hdr["metric"], hdr["ntotal"],
                                                            hdr["is_trained"])
    assert np.array_equal(g.reconstruct_n(0, g.ntotal), x)
    r = g.search(x, 5)
    g.close()
    Dr, Ir = oracle.flat_search(x, x, 5, oracle.IP)
    assert_knn_parity(r.distances, r.ids, Dr, Ir, 1)
    assert np.array_equal(r.ids[:, 0], np.arange(hdr["ntotal"]))  # self top-1


def test_faiss_golden_and_roundtrip(vs, tmp_path):
    g = vs.GpuIndexFlat.load(GOLDEN)
    assert (g.d, int(g.metric), g.ntotal, g.is_trained) == (2, 0, 1, True)
    assert np.array_equal(g.reconstruct(0), [3.0, 4.0])
    assert g.search(np.array([[0.0, 0.0]], np.float32), 1).distances[0, 0] == 25.0
    g.close()
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3001, 33)).astype(np.float32)
    for metric in (0, 1):
        blob = vio.write_faiss_flat(33, metric, x)
        p = tmp_path / f"f{metric}.bin"
        p.write_bytes(blob)
        g = vs.GpuIndexFlat.load(str(p), storage="f32")
        assert int(g.metric) == metric and g.ntotal == 3001
        r = g.search(x[:20], 7)
        g.close()
        Dr, Ir = oracle.flat_search(x, x[:20], 7, metric)
        assert_knn_parity(r.distances, r.ids, Dr, Ir, metric)


def test_malformed_blobs_rejected(vs):
    with pytest.raises(ValueError, match="bad magic"):
        vs.GpuIndexFlat.load(b"\x00" * 64)
    bad_metric = bytearray(GOLDEN)
    bad_metric[33] = 7
    with pytest.raises(ValueError, match="Unsupported FAISS metric code 7"):
        vs.GpuIndexFlat.load(bytes(bad_metric))
    bad_size = bytearray(GOLDEN)
    bad_size[37] = 9
    with pytest.raises(ValueError, match="IndexFlat payload size 9 != ntotal\\*d\\*4 = 8"):
        vs.GpuIndexFlat.load(bytes(bad_size))
    with pytest.raises(ValueError, match="truncated"):
        vs.GpuIndexFlat.load(GOLDEN[:50])
    fd = vio.write_faisdart_flat(4, 1, np.ones((3, 4), np.float32))
    bad = bytearray(fd)
    bad[20] = 5  # metric code
    with pytest.raises(ValueError, match="Unknown metric code 5"):
        vs.GpuIndexFlat.load(bytes(bad))
    kind = bytearray(fd)
    kind[12] = 2  # not IndexFlat
    with pytest.raises(NotImplementedError):
        vs.GpuIndexFlat.load(bytes(kind))
