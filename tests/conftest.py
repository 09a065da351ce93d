"""Test configuration.

Tests marked ``gpu`` need an MI355X (they run the HIP library); everything
else runs on the CPU: the oracle and its pinning, the host-side cache logic,
and the C ABI's argument validation (which returns before any HIP call).
"""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "custom-inference-engine_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="GPU required")
    for item in items:
        if item.get_closest_marker("gpu"):
            item.add_marker(skip)
