"""Shared pytest setup: import paths, the ``gpu`` marker and seeded helpers.

GPU tests (``-m gpu``) call the HIP kernels through the C ABI / dispatcher on
``cuda:0`` and check them against the CPU oracle in ``oracle/``; CPU tests
(``-m "not gpu"``) pin the oracle and exercise the host-side logic.
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "maba-v2-architecture_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# Every GPU test must exercise the HIP path: never let the dispatcher fall back.
os.environ.setdefault("MABA_STRICT_BACKEND", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950) and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available() and bool(getattr(torch.version, "hip", None))
    except Exception:
        return False


@pytest.fixture
def dev():
    import torch
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")
