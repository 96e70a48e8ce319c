"""Shared test setup: import paths, the ``gpu`` marker, precision policy and helpers."""

import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
for path in (ROOT, ROOT / "torch-convnd_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

GPU_AVAILABLE = torch.cuda.is_available() and torch.version.hip is not None


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")
    config.addinivalue_line("markers", "portable: runs without the native libraries")


def pytest_collection_modifyitems(config, items):
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords and not GPU_AVAILABLE:
            item.add_marker(skip)


@pytest.fixture(scope="session", autouse=True)
def precision_policy():
    """No TF32 anywhere, and bounded CPU threads for the portable comparisons."""
    previous = (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32)
    threads = torch.get_num_threads()
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_num_threads(min(threads, int(os.environ.get("TORCH_CONVND_TEST_THREADS", "8"))))
    yield
    torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32 = previous
    torch.set_num_threads(threads)


@pytest.fixture
def deterministic_algorithms():
    previous = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(previous)
