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
