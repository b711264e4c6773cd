from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built native library")
    config.addinivalue_line("markers", "slow: long-running")


def pytest_collection_modifyitems(config, items) -> None:
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for it in gpu_items:
        it.add_marker(skip)


@pytest.fixture
def dev() -> torch.device:
    return torch.device("cuda:0")


def pytest_runtest_setup(item) -> None:
    # Name the case before any GPU work, so a run that dies still says where.
    if "gpu" in item.keywords:
        print(f"\n[gpu-case] {item.nodeid}", flush=True)
