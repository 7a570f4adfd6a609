"""Test configuration: repo root on sys.path and the ``gpu`` marker.

``-m "not gpu"`` runs on a CPU-only host (oracle, host logic, C-ABI surface);
``-m gpu`` needs an MI355X and calls the HIP library through the C ABI.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built HIP library")


def gpu_available():
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch missing
        return False


@pytest.fixture(scope="session")
def device():
    if not gpu_available():
        pytest.skip("GPU required")
    return "cuda:0"
