"""Shared pytest setup: repo root on sys.path, the `gpu` marker, seeded inputs."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def device():
    """cuda:0 with the native library loaded; fails (not skips) if the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import fast_dl_amd.capi as capi

    capi.load_library()
    return torch.device("cuda:0")


def rng(seed: int) -> np.random.Generator:
    """All synthetic inputs come from numpy's PCG64 with a recorded seed."""
    return np.random.default_rng(seed)
