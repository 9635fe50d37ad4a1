"""MI355X flat exact nearest-neighbour search: Python mirror of the reference's
vector-store API on this path (lib/core/vector_store/{index,index_flat,
gpu_index_flat,kmeans}.dart) over libvs_hip.so."""
from ._native import NativeLibraryError, VsError, device_count, device_name, load
from .gpu_index_flat import GpuIndexFlat, IndexFlatIP, IndexFlatL2
from .index import Index, Metric, RangeSearchResult, SearchResult, recall_at_k
from .ivf import IndexIVFFlat
from .wrappers import IndexIDMap, IndexPreTransform, IndexRefineFlat, IndexShards, L2NormTransform
from .kmeans import Kmeans, KmeansResult, kmeans_step

__all__ = [
    "GpuIndexFlat", "IndexFlatL2", "IndexFlatIP", "Index", "Metric", "SearchResult",
    "RangeSearchResult", "recall_at_k", "IndexIVFFlat", "IndexIDMap", "IndexPreTransform",
    "IndexRefineFlat", "IndexShards", "L2NormTransform", "Kmeans", "KmeansResult", "kmeans_step", "load",
    "device_count", "device_name", "NativeLibraryError", "VsError",
]
