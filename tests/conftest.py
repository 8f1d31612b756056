"""Shared test setup: import paths, the ``gpu`` marker, seeded inputs."""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "dattri-llm_amd")
for _p in (PKG_ROOT, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def rel_err(got, ref) -> float:
    """Normwise relative error max|got - ref| / max|ref| (entrywise relative
    error is ill-posed for near-zero scores)."""
    import numpy as np

    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = float(np.abs(ref).max()) if ref.size else 1.0
    return float(np.abs(got - ref).max() / (denom if denom > 0 else 1.0)) if ref.size else 0.0
