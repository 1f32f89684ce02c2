"""Test configuration: import paths, the ``gpu`` marker and shared helpers.

Tests marked ``gpu`` need a ROCm GPU and the built HIP library; everything
else runs on the CPU.  On a GPU run a missing library is an error (the
backend never falls back), so ``gpu`` tests fail rather than skip in that
case.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = REPO_ROOT / "nano-vllm-multimodal_amd"
for path in (REPO_ROOT, PACKAGE_ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libnanokv.so")


def gpu_available() -> bool:
    import torch

    return torch.version.hip is not None and torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not gpu_available():
        pytest.skip("no ROCm GPU visible")
    from nanokv import _lib

    _lib.load_library()  # raises (test error) if the library is missing
    return torch.device("cuda", 0)
