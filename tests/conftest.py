"""Shared fixtures: seeded inputs shaped like the BASELINE configs, GPU gate."""

from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    return torch.device("cuda")


from smaq_amd.synthetic import spectral_sigma  # noqa: E402,F401


def sample_keys(n: int, d: int = 128, seed: int = 1, sigma_seed: int = 0) -> torch.Tensor:
    """n keys ~ N(0, Sigma) (fp32, CPU); see smaq_amd.synthetic."""
    _, u, lam = spectral_sigma(d, sigma_seed)
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(n, d, generator=g)
    return (z * lam.sqrt()) @ u.T
