"""pytest configuration: the `gpu` marker, import paths and shared fixtures.

The product package lives in torch-projectors_amd/ (import name
`torch_projectors`, as in the reference); the oracle binding in oracle/.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "torch-projectors_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Skip when no GPU is visible; the HIP library must then load (no fallback)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import torch_projectors  # noqa: F401  (raises ImportError when the native library is missing)
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def hip(gpu):
    """The C-ABI driver of tests/hip_path.py."""
    from tests import hip_path
    return hip_path


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    return O
