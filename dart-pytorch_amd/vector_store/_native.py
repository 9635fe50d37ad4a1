"""Loader of libvs_hip.so, the gfx950 flat-search library (C ABI in include/vs_hip.h).

Resolution order mirrors the reference's native-library lookup
(lib/core/tensor/cuda_engine.dart:428-455): the DART_PYTORCH_VS_LIB
environment variable, then the package's own lib/ directory.  There is no
CPU fallback: a missing or unloadable library raises NativeLibraryError.
"""
from __future__ import annotations

import ctypes
import os

VS_OK = 0
VS_ERR_INVALID = 1
VS_ERR_OOM = 2
VS_ERR_HIP = 3
VS_ERR_UNSUPPORTED = 4
VS_ERR_NONFINITE = 5
VS_ERR_NO_DEVICE = 6

VS_DTYPE_F32 = 0
VS_DTYPE_BF16 = 1
VS_STORAGE_F32 = 0
VS_STORAGE_BF16 = 1
VS_STORAGE_AUTO = 2

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "lib", "libvs_hip.so")

# every entry point of include/vs_hip.h
EXPORTED = [
    "vs_index_create", "vs_index_destroy", "vs_index_reserve", "vs_index_reset",
    "vs_index_ntotal", "vs_index_d", "vs_index_metric", "vs_index_storage",
    "vs_index_add", "vs_index_add_device", "vs_index_reconstruct", "vs_index_remove_ids",
    "vs_index_load_flat", "vs_index_load_flat_buffer",
    "vs_index_search", "vs_index_search_device", "vs_index_search_device_noalloc",
    "vs_index_search_subsets", "vs_index_score_all",
    "vs_index_range_search", "vs_range_result_free",
    "vs_index_self_join", "vs_pairs_free", "vs_kmeans_step", "vs_last_error",
    "vs_dev_alloc", "vs_dev_free", "vs_dev_upload", "vs_dev_download", "vs_dev_copy", "vs_dev_probe",
    "vs_dev_mfma_chain",
    "vs_device_count",
    "vs_device_name", "vs_gen_normal", "vs_prof_enable", "vs_prof_get", "vs_prof_reset",
    "vs_index_sync", "vs_index_set_option",
]


class NativeLibraryError(RuntimeError):
    """libvs_hip.so is missing or failed to load."""


class VsError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[vs error {code}] {msg}")
        self.code = code


class RangeSearchC(ctypes.Structure):
    _fields_ = [
        ("nq", ctypes.c_int64),
        ("lims", ctypes.POINTER(ctypes.c_int64)),
        ("D", ctypes.POINTER(ctypes.c_float)),
        ("I", ctypes.POINTER(ctypes.c_int32)),
    ]


class PairsC(ctypes.Structure):
    _fields_ = [
        ("npairs", ctypes.c_int64),
        ("i", ctypes.POINTER(ctypes.c_int32)),
        ("j", ctypes.POINTER(ctypes.c_int32)),
        ("s", ctypes.POINTER(ctypes.c_float)),
    ]


_lib = None


def library_path() -> str:
    return os.environ.get("DART_PYTORCH_VS_LIB") or LIB_PATH


def load() -> ctypes.CDLL:
    """Load and bind libvs_hip.so (once)."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise NativeLibraryError(
            f"libvs_hip.so not found at {path}; build it with __graft_entry__.build() "
            "or `make -C dart-pytorch_amd/csrc`")
    try:
        L = ctypes.CDLL(path)
    except OSError as e:  # pragma: no cover - depends on the environment
        raise NativeLibraryError(f"failed to load {path}: {e}") from e
    p = ctypes.c_void_p
    i64 = ctypes.c_int64
    i32 = ctypes.c_int
    pp = ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "vs_index_create": ([i32, i64, i32, i32, pp], i32),
        "vs_index_destroy": ([p], None),
        "vs_index_reserve": ([p, i64], i32),
        "vs_index_reset": ([p], i32),
        "vs_index_ntotal": ([p], i64),
        "vs_index_d": ([p], i64),
        "vs_index_metric": ([p], i32),
        "vs_index_storage": ([p], i32),
        "vs_index_add": ([p, p, i32, i64], i32),
        "vs_index_add_device": ([p, p, i32, i64], i32),
        "vs_index_reconstruct": ([p, i64, i64, p], i32),
        "vs_index_remove_ids": ([p, p, i64, ctypes.POINTER(ctypes.c_int64)], i32),
        "vs_index_load_flat": ([i32, ctypes.c_char_p, i32, pp, ctypes.POINTER(i32)], i32),
        "vs_index_load_flat_buffer": ([i32, p, i64, i32, pp, ctypes.POINTER(i32)], i32),
        "vs_index_search": ([p, p, i32, i64, i64, p, p], i32),
        "vs_index_search_device": ([p, p, i32, i64, i64, p, p], i32),
        "vs_index_search_device_noalloc": ([p, p, i32, i64, i64, p, p], i32),
        "vs_index_search_subsets": ([p, p, i32, i64, i64, p, i64, p, p, i64, p, p], i32),
        "vs_index_score_all": ([p, p, p], i32),
        "vs_index_range_search": ([p, p, i32, i64, ctypes.c_double,
                                   ctypes.POINTER(ctypes.POINTER(RangeSearchC))], i32),
        "vs_range_result_free": ([ctypes.POINTER(RangeSearchC)], None),
        "vs_index_self_join": ([p, ctypes.c_double, ctypes.POINTER(ctypes.POINTER(PairsC))], i32),
        "vs_pairs_free": ([ctypes.POINTER(PairsC)], None),
        "vs_kmeans_step": ([p, p, i64, i64, p, i64, p, p, p, ctypes.POINTER(ctypes.c_double)], i32),
        "vs_last_error": ([], ctypes.c_char_p),
        "vs_dev_alloc": ([i32, i64, pp], i32),
        "vs_dev_free": ([i32, p], i32),
        "vs_dev_upload": ([i32, p, p, i64], i32),
        "vs_dev_download": ([i32, p, p, i64], i32),
        "vs_dev_copy": ([i32, p, p, i64], i32),
        "vs_dev_probe": ([i32, i32, i64, ctypes.POINTER(ctypes.c_double)], i32),
        "vs_dev_mfma_chain": ([i32, i32, i64, i64, p, p, p, p], i32),
        "vs_device_count": ([ctypes.POINTER(ctypes.c_int)], i32),
        "vs_device_name": ([i32, ctypes.c_char_p, i64], i32),
        "vs_gen_normal": ([i32, p, i32, i64, i64, ctypes.c_uint64, ctypes.c_uint64, i32], i32),
        "vs_prof_enable": ([p, i32], i32),
        "vs_prof_get": ([p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64),
                         ctypes.POINTER(ctypes.c_double)], i32),
        "vs_prof_reset": ([p], i32),
        "vs_index_sync": ([p], i32),
        "vs_index_set_option": ([p, ctypes.c_char_p, i64], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return _lib


def last_error() -> str:
    return load().vs_last_error().decode(errors="replace")


def check(rc: int) -> None:
    """Raise the Python counterpart of a non-zero status.

    VS_ERR_INVALID maps to ValueError (the reference throws ArgumentError /
    RangeError), VS_ERR_UNSUPPORTED to NotImplementedError (UnsupportedError),
    everything else to VsError."""
    if rc == VS_OK:
        return
    msg = last_error()
    if rc == VS_ERR_INVALID:
        raise ValueError(msg)
    if rc == VS_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise VsError(rc, msg)


def device_count() -> int:
    c = ctypes.c_int(0)
    rc = load().vs_device_count(ctypes.byref(c))
    return c.value if rc == VS_OK else 0


def device_name(device: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    check(load().vs_device_name(device, buf, 256))
    return buf.value.decode()


class DeviceBuffer:
    """A raw device allocation (bench and tests keep inputs resident in HBM)."""

    def __init__(self, nbytes: int, device: int = 0):
        self.device = device
        self.nbytes = int(nbytes)
        ptr = ctypes.c_void_p()
        check(load().vs_dev_alloc(device, self.nbytes, ctypes.byref(ptr)))
        self.ptr = ptr

    def upload(self, host) -> None:
        import numpy as np

        a = np.ascontiguousarray(host)
        assert a.nbytes <= self.nbytes
        check(load().vs_dev_upload(self.device, self.ptr, a.ctypes.data_as(ctypes.c_void_p), a.nbytes))

    def download(self, host) -> None:
        assert host.flags["C_CONTIGUOUS"] and host.nbytes <= self.nbytes
        check(load().vs_dev_download(self.device, host.ctypes.data_as(ctypes.c_void_p), self.ptr,
                                     host.nbytes))

    def free(self) -> None:
        if self.ptr:
            load().vs_dev_free(self.device, self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):  # pragma: no cover - interpreter teardown order
        try:
            self.free()
        except Exception:
            pass
