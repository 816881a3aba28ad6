"""Shared pytest setup: repo root on sys.path, the `gpu` marker, GPU availability."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); runs the HIP kernels")


def _gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
