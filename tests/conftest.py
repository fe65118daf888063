"""Shared pytest set-up: the `gpu` marker, import paths for the package and the oracle, and
fixtures for device tests."""

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for path in (REPO / "oxide-beta_amd", REPO / "oracle", REPO):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def rng():
    import numpy as np

    return np.random.default_rng(0x6F786964)


@pytest.fixture(scope="session")
def module():
    """The HIP launchers on cuda:0 (fails loudly when the library or the GPU is missing)."""
    import torch

    import oxide_hip

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return oxide_hip.load_kernels(0)


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")
