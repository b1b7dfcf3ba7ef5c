"""Shared pytest setup: the `gpu` marker, import paths, and seeded data helpers."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("kern-k3_amd", "oracle", "tests"):
    p = os.path.join(REPO, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def ctx():
    """k3h context over the built code objects (GPU tests only)."""
    import torch
    import k3h
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    c = k3h.Ctx()
    yield c
    c.close()
