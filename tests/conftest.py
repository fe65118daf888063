"""Shared pytest set-up: the `gpu` marker and import paths for the package and the oracle."""

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
