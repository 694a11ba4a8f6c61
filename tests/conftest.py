"""Shared pytest configuration.

Markers: ``gpu`` (needs a ROCm device and the built libkernelforge_hip.so) and
``slow``. GPU tests skip on a host without a device, as in the reference
(tests/conftest.py:7-19); on a GPU host a missing library is a failure, not a
skip.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")
    config.addinivalue_line("markers", "slow: long-running")


def _gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU attached")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def device():
    import torch

    return torch.device("cuda")


@pytest.fixture
def mi355x_caps():
    from kernelforge.runtime.env import MI355X_CAPS

    return MI355X_CAPS
