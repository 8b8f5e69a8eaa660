"""Test configuration: the repo root on sys.path and the `gpu` marker.

`-m "not gpu"` tests run on any host (oracle against the reference's known
answers, host logic, C-ABI exports). `-m gpu` tests are the parity tests:
they call libferric_hip.so through its C ABI on an MI355X and compare with
the CPU oracle.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
