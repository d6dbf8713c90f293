"""Shared pytest setup.

``-m gpu`` tests run on an MI355X and call the HIP library through the C ABI;
everything else runs on the CPU (oracle checks, host logic, library loading).
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HAS_GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    if HAS_GPU:
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    return torch.device("cuda", 0)


def announce(msg: str) -> None:
    """Name the case before a GPU step, so a crash log says what ran."""
    print(f"[case] {msg}", flush=True)
