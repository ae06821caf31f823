"""Shared pytest setup: import paths, the `gpu` marker, and fixtures.

CPU tests (`-m "not gpu"`) cover the oracle against the golden fixtures, the
host-side logic of the native libraries and their exported C-ABI.  GPU tests
(`-m gpu`) are the parity tests proper and run on an MI355X.
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "jax-mlx-plugin_amd", REPO / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def oracle():
    import oracle_api

    return oracle_api


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    return dict(np.load(REPO / "tests" / "golden" / "fixtures.npz"))


@pytest.fixture(scope="session")
def cuda():
    """The torch module with a visible GPU; skips where there is none."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch
