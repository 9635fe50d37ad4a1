"""Flat-index on-disk formats, loaded straight into a GPU index (load_flat,
through the library's loader) and read / written on the host (the
read_* / write_* helpers, used by the tests as the format's checker).

FAISDART (the reference's own format, index_io.dart:8-26): magic
'FAISDART', u32 version (1), u32 kind (0x01 = IndexFlat), then the common
header d u32, metric u32 (0 = L2, 1 = IP, index_io.dart:233), ntotal u32,
isTrained u8, then ntotal*d little-endian fp32 (IndexFlat.writeTo,
index_flat.dart:165-188).

FAISS binary IndexFlat (faiss_io.dart:1501-1522 write, :1690-1716 read):
fourcc 'IxF2' (L2) / 'IxFI' (IP), d i32, ntotal i64, two legacy i64 (1<<20),
is_trained u8, metric i32 (FAISS codes: 0 = IP, 1 = L2, faiss_io.dart:396-402),
then a byte vector (u64 size + bytes) holding the row-major fp32 matrix.

The layouts are fixed by the files they read, so the field order here is
necessarily the reference's.
"""
from __future__ import annotations

import struct

import numpy as np

from .index import Metric

FAISDART_MAGIC = b"FAISDART"
KIND_FLAT = 0x01
FOURCC_FLAT_L2 = b"IxF2"
FOURCC_FLAT_IP = b"IxFI"
FOURCC_FLAT = b"IxFl"


def _bytes(src) -> bytes:
    if isinstance(src, (bytes, bytearray, memoryview)):
        return bytes(src)
    with open(src, "rb") as f:
        return f.read()


def read_faisdart_flat(src):
    """Returns (header dict, float32 (ntotal, d) array) of a FAISDART IndexFlat blob."""
    b = _bytes(src)
    if len(b) < 29 or b[:8] != FAISDART_MAGIC:
        raise ValueError("not a FAISDART blob (bad magic)")
    version, kind = struct.unpack_from("<II", b, 8)
    if version != 1:
        raise ValueError(f"unsupported FAISDART version {version}")
    if kind != KIND_FLAT:
        raise ValueError(f"FAISDART kind {kind:#x} is not IndexFlat")
    d, metric, ntotal, trained = struct.unpack_from("<IIIB", b, 16)
    if metric not in (0, 1):
        raise ValueError(f"Unknown metric code {metric}")
    need = 29 + 4 * ntotal * d
    if len(b) < need:
        raise ValueError(f"truncated FAISDART payload: {len(b)} < {need} bytes")
    x = np.frombuffer(b, dtype="<f4", count=ntotal * d, offset=29).reshape(ntotal, d).astype(np.float32)
    return {"d": d, "metric": metric, "ntotal": ntotal, "is_trained": bool(trained)}, x


def write_faisdart_flat(d: int, metric: int, x: np.ndarray, is_trained: bool = True) -> bytes:
    x = np.ascontiguousarray(x, dtype="<f4")
    hdr = FAISDART_MAGIC + struct.pack("<II", 1, KIND_FLAT)
    hdr += struct.pack("<IIIB", d, int(metric), x.shape[0], 1 if is_trained else 0)
    return hdr + x.tobytes()


def read_faiss_flat(src):
    """Returns (header dict, float32 (ntotal, d) array) of a FAISS IndexFlat blob."""
    b = _bytes(src)
    tag = b[:4]
    if tag not in (FOURCC_FLAT_L2, FOURCC_FLAT_IP, FOURCC_FLAT):
        raise ValueError(f"unsupported FAISS fourcc {tag!r}")
    d, = struct.unpack_from("<i", b, 4)
    ntotal, _, _ = struct.unpack_from("<qqq", b, 8)
    trained, = struct.unpack_from("<B", b, 32)
    fmetric, = struct.unpack_from("<i", b, 33)
    if fmetric not in (0, 1):
        raise ValueError(f"unsupported FAISS metric {fmetric}")
    nbytes, = struct.unpack_from("<Q", b, 37)
    if nbytes != ntotal * d * 4:
        raise ValueError(f"IndexFlat payload size {nbytes} != ntotal*d*4 = {ntotal * d * 4}")
    x = np.frombuffer(b, dtype="<f4", count=ntotal * d, offset=45).reshape(ntotal, d).astype(np.float32)
    metric = int(Metric.l2) if fmetric == 1 else int(Metric.innerProduct)
    return {"d": d, "metric": metric, "ntotal": ntotal, "is_trained": bool(trained)}, x


def write_faiss_flat(d: int, metric: int, x: np.ndarray, is_trained: bool = True) -> bytes:
    x = np.ascontiguousarray(x, dtype="<f4")
    tag = FOURCC_FLAT_L2 if int(metric) == int(Metric.l2) else FOURCC_FLAT_IP
    fmetric = 1 if int(metric) == int(Metric.l2) else 0
    out = tag + struct.pack("<iqqqBi", d, x.shape[0], 1 << 20, 1 << 20, 1 if is_trained else 0, fmetric)
    payload = x.tobytes()
    return out + struct.pack("<Q", len(payload)) + payload


def load_flat(src, storage: str = "auto", device: int = 0):
    """A GpuIndexFlat holding the vectors of a FAISDART or FAISS IndexFlat
    blob (a path, or bytes): the library parses the header and streams the
    rows into HBM (vs_index_load_flat / vs_index_load_flat_buffer); the host
    never holds the whole payload when given a path."""
    import ctypes

    from . import _native as N
    from .gpu_index_flat import GpuIndexFlat

    lib = N.load()
    h = ctypes.c_void_p()
    trained = ctypes.c_int(0)
    code = GpuIndexFlat._STORAGE[storage]
    if isinstance(src, (bytes, bytearray, memoryview)):
        buf = bytes(src)
        N.check(lib.vs_index_load_flat_buffer(device, buf, len(buf), code, ctypes.byref(h),
                                              ctypes.byref(trained)))
    else:
        N.check(lib.vs_index_load_flat(device, str(src).encode(), code, ctypes.byref(h),
                                       ctypes.byref(trained)))
    g = GpuIndexFlat._adopt(h, device)
    g.is_trained = bool(trained.value)
    return g
