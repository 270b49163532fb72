"""Shared pytest setup: import paths, the ``gpu`` marker and seeded inputs."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for _p in (str(ROOT / "triton-muonadamw_amd"), str(ROOT)):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; a GPU test without one fails loudly instead of skipping."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("this test needs a ROCm GPU")
    return torch.device("cuda:0")
