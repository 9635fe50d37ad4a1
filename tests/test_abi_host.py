"""CPU-tier checks of the boundary and host logic (no GPU needed):
the C-ABI library loads and exports every entry point include/vs_hip.h
declares; file formats match the reference's golden bytes; the parity
helper rejects planted mistakes."""
import ctypes
import os
import re

import numpy as np
import pytest

from _parity import assert_knn_parity, assert_range_parity

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    src = open(os.path.join(ROOT, "include", "vs_hip.h")).read()
    return sorted(set(re.findall(r"VS_API\s+[\w\s\*]+?\b(vs_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from vector_store import _native

    lib = _native.load()  # raises NativeLibraryError when missing: no fallback
    syms = header_symbols()
    assert len(syms) >= 30
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in vs_hip.h but not exported"
    assert sorted(_native.EXPORTED) == syms


def test_missing_library_fails_loudly(monkeypatch):
    from vector_store import _native

    monkeypatch.setenv("DART_PYTORCH_VS_LIB", "/nonexistent/libvs_hip.so")
    monkeypatch.setattr(_native, "_lib", None)
    with pytest.raises(_native.NativeLibraryError):
        _native.load()


def test_faiss_flat_golden_bytes():
    """The 53-byte IxF2 blob of IndexFlatL2(2) holding [3, 4]
    (vector_store_test.dart:1018-1093)."""
    from vector_store import io as vio

    golden = bytes([0x49, 0x78, 0x46, 0x32, 0x02, 0, 0, 0, 0x01, 0, 0, 0, 0, 0, 0, 0,
                    0, 0, 0x10, 0, 0, 0, 0, 0, 0, 0, 0x10, 0, 0, 0, 0, 0, 0x01,
                    0x01, 0, 0, 0, 0x08, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0x40, 0x40, 0, 0, 0x80, 0x40])
    assert len(golden) == 53
    assert vio.write_faiss_flat(2, 0, np.array([[3.0, 4.0]], np.float32)) == golden
    hdr, x = vio.read_faiss_flat(golden)
    assert hdr == {"d": 2, "metric": 0, "ntotal": 1, "is_trained": True}
    assert np.array_equal(x, [[3.0, 4.0]])
    ip = vio.write_faiss_flat(2, 1, np.array([[3.0, 4.0]], np.float32))
    assert ip[:4] == b"IxFI" and ip[33:37] == b"\x00\x00\x00\x00"  # FAISS metric 0 = IP


def test_faisdart_roundtrip_and_fixture():
    from vector_store import io as vio

    path = os.path.join(ROOT, "tests", "golden", "docs_index.bin")
    raw = open(path, "rb").read()
    hdr, x = vio.read_faisdart_flat(raw)
    assert (hdr["d"], hdr["metric"], hdr["ntotal"], hdr["is_trained"]) == (384, 1, 20, True)
    assert np.allclose(np.linalg.norm(x, axis=1), 1.0, atol=1e-6)
    assert vio.write_faisdart_flat(384, 1, x) == raw
    with pytest.raises(ValueError):
        vio.read_faisdart_flat(b"\x00" * 64)  # bad magic (vector_store_test.dart:298)


def test_parity_helper_rejects_planted_mistakes():
    D = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    I = np.array([[10, 11, 12, 13]], np.int32)
    assert_knn_parity(D, I, D, I, 0)
    with pytest.raises(AssertionError):  # swapped ids of distinct distances
        assert_knn_parity(D, I[:, [1, 0, 2, 3]], D, I, 0)
    with pytest.raises(AssertionError):  # a wrong distance
        assert_knn_parity(D + np.float32([0, 0, 1e-3, 0]), I, D, I, 0)
    with pytest.raises(AssertionError):  # a dropped neighbour
        assert_knn_parity(D, np.array([[10, 11, 99, 13]], np.int32), D, I, 0)
    Dt = np.array([[1.0, 2.0, 2.0, 4.0]], np.float32)  # tie: order may differ
    assert_knn_parity(Dt, I[:, [0, 2, 1, 3]], Dt, I, 0)
    # the last tie group may continue past k: row 2 ties row 1 at distance 1
    # (L2 to the query 0), so either may fill the last slot -- but an extra id
    # must really lie at the reported distance
    xb = np.array([[0.0], [1.0], [1.0], [3.0]], np.float32)
    xq = np.zeros((1, 1), np.float32)
    Dk = np.array([[0.0, 1.0]], np.float32)
    assert_knn_parity(Dk, np.array([[0, 2]], np.int32), Dk, np.array([[0, 1]], np.int32), 0,
                      xb=xb, xq=xq)
    with pytest.raises(AssertionError):  # row 3 is at distance 9, not 1
        assert_knn_parity(Dk, np.array([[0, 3]], np.int32), Dk, np.array([[0, 1]], np.int32), 0,
                          xb=xb, xq=xq)
    lims = np.array([0, 2]); Dr = np.array([1.0, 2.0], np.float32); Ir = np.array([3, 5], np.int32)
    assert_range_parity(lims, Dr, Ir, lims, Dr, Ir)
    with pytest.raises(AssertionError):
        assert_range_parity(lims, Dr, np.array([3, 6], np.int32), lims, Dr, Ir)


def test_synthetic_generators():
    from vector_store import synthetic as syn

    a = syn.normal_unit(100, 64, 1, 0)
    assert np.allclose(np.linalg.norm(a.astype(np.float64), axis=1), 1.0, atol=1e-6)
    assert np.array_equal(a, syn.normal_unit(100, 64, 1, 0))  # seeded
    g = syn.int_grid(50, 8, 1, 0)
    assert g.min() >= 0 and g.max() <= 255 and np.all(g == np.round(g))
    # bf16 spacing at 1.0 is 2^-7: 1 + 2^-7 is exact; 1 + 2^-8 is a tie that
    # rounds to even (1.0); 1 + 3 * 2^-8 is a tie that rounds up to 1 + 2^-6
    b = syn.to_bf16_bits(np.array([1.0, 1.0078125, 1.00390625, 1.01171875, -2.5], np.float32))
    assert list(syn.bf16_bits_to_f32(b)) == [1.0, 1.0078125, 1.0, 1.015625, -2.5]
    x = syn.dedup_set(1000, 16, 0.05, 0.01, 3)
    assert x.shape == (1000, 16)


def test_l2_normalize_is_the_reference_order():
    """L2NormTransform.apply (l2_norm_transform.dart:23-46) restated with
    scalar loops: s += v * v in dimension order, inv = 1 / sqrt(s),
    fp32(v * inv); a zero row stays zero.  The host normaliser must match
    it bit for bit (a pairwise or reordered sum differs in the last bits of
    some rows)."""
    from vector_store import synthetic as syn
    from vector_store.wrappers import L2NormTransform

    g = np.random.default_rng(8)
    x = g.standard_normal((40, 301)).astype(np.float32)
    x[7] = 0.0
    want = np.empty_like(x)
    for i, row in enumerate(x):
        s = 0.0
        for v in row:
            s = s + float(v) * float(v)
        norm = float(np.sqrt(s))
        want[i] = [np.float32(float(v) * (1.0 / norm)) if norm > 0 else 0.0 for v in row]
    assert np.array_equal(syn.l2_normalize(x).view(np.uint32), want.view(np.uint32))
    assert np.array_equal(L2NormTransform(301).apply(x).view(np.uint32), want.view(np.uint32))
    assert not want[7].any()
