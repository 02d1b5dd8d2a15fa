"""Shared pytest setup: import paths and the ``gpu`` marker.

GPU tests are marked ``gpu`` and skip themselves when no GPU is visible;
``python -m pytest -m "not gpu"`` runs everything that needs only the CPU.
"""
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for path in (REPO, REPO / "paged-decode-lab_amd", REPO / "tests" / "golden"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (gfx950) and the built HIP libraries")


def gpu_available():
    try:
        import torch
    except ImportError:
        return False
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


def announce(message):
    """Print and flush a case description before a GPU step."""
    print(message, flush=True)
    sys.stdout.flush()
    os.fsync(sys.stdout.fileno()) if hasattr(sys.stdout, "fileno") and sys.stdout.isatty() else None
