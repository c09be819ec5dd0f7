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


@pytest.fixture(scope="session")
def ctx():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vectorstorekit_amd.engine import Context

    c = Context(0)
    yield c
    c.close()
