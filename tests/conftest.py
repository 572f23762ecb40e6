"""Test configuration: registers the ``gpu`` marker and puts the repo on sys.path.

``-m "not gpu"`` runs the CPU suite (oracle pinning, host logic, library
symbols, rejection paths); ``-m gpu`` runs the HIP-vs-oracle parity tests on an
MI355X.  GPU tests skip (never pass) when no GPU is visible.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

_TESTS = Path(__file__).resolve().parent
sys.path.insert(0, str(_TESTS))
sys.path.insert(0, str(_TESTS.parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP kernels run)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
