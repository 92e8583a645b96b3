"""Test setup: the package root and the oracle on sys.path, the ``gpu`` marker, and shared fixtures.

``-m "not gpu"`` runs the oracle against the reference's known answers and golden vectors, the host logic (packs,
registry, planning) and the C-ABI export check; ``-m gpu`` runs the HIP kernels through the C ABI against the
oracle on an MI355X.
"""

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "lithos-metal_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libmi355.so")


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from monolith_mi355.runtime import hip
    hip.load()                                   # fails loudly when the library is missing
    return torch


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
