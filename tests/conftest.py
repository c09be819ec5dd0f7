"""pytest setup: the repo root on sys.path, the ``gpu`` marker, and a
session-wide HIP context for GPU tests."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvsk_hip.so)")


@pytest.fixture(scope="session", autouse=True)
def _torch_initialises_hip_first(request):
    """GPU runs: torch initialises the HIP runtime before the library does
    (the library opened first leaves torch.cuda.is_available() False in
    this image, which would skip every test that asks torch for the GPU)."""
    if request.config.getoption("-m") and "not gpu" not in request.config.getoption("-m"):
        import torch

        torch.cuda.is_available()
    yield


@pytest.fixture(scope="session")
def ctx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vectorstorekit_amd.engine import Context

    c = Context(0)
    yield c
    c.close()
