"""pytest configuration: the `gpu` marker, import paths and shared fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "asc-devkit_clone_amd"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X); parity tests through the C ABI")


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib

    oracle_lib.lib()
    return oracle_lib


@pytest.fixture(scope="session")
def ascq_gpu():
    """The ascq binding with a live GPU.  On a GPU run a missing device or library is an error, not a skip."""
    import torch

    import ascq

    if not torch.cuda.is_available():
        raise RuntimeError("GPU test run without a visible GPU")
    ascq.lib()
    torch.cuda.init()
    return ascq


def seeded(seed: int):
    import numpy as np

    return np.random.default_rng(seed)
