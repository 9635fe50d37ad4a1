import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "dart-pytorch_amd"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvs_hip.so on cuda:0)")


@pytest.fixture(scope="session")
def vs():
    """The product package; GPU tests fail loudly if libvs_hip.so or the GPU is missing."""
    import vector_store

    vector_store.load()
    if vector_store.device_count() < 1:
        pytest.fail("no HIP device visible to libvs_hip.so")
    return vector_store


@pytest.fixture
def opts(monkeypatch):
    """opts(name=value, ...) forces planner options (vs_index_set_option) on
    every index the test creates from then on; restored afterwards."""
    from vector_store import gpu_index_flat

    def set_(**kw):
        for name, value in kw.items():
            monkeypatch.setitem(gpu_index_flat.DEFAULT_OPTIONS, name, int(value))

    return set_
