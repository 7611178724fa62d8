"""Shared test setup: import paths, the `gpu` marker and common helpers."""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT / "nsa-test_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

FIXTURES = ROOT / "tests" / "golden" / "fixtures"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libnsa_hip.so")


def rel_err(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))


def load_fixture(name):
    return np.load(FIXTURES / f"{name}.npz", allow_pickle=False)


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
