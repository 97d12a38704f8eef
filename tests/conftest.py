"""pytest configuration: the `gpu` marker and shared fixtures.

Tests marked `gpu` need an MI355X and the built library; everything else runs on the CPU (the checker under
oracle/, host-side logic, and the C ABI's argument validation, which returns before touching a device).
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and firefly_amd/libffkv.so")


def _has_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a GPU is present; returns the torch device."""
    if not _has_gpu():
        pytest.skip("no GPU")
    import torch

    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ff():
    import firefly_amd

    return firefly_amd
