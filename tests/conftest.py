"""Shared test setup: the `gpu` marker, repo-root imports, and the device gate.

CPU tests (`-m "not gpu"`) cover the oracle against golden vectors and library routines,
the host logic of the façades and the C-ABI library's exports. GPU tests (`-m gpu`) are
the parity tests of the HIP kernels against the oracle, called through the C-ABI.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
