"""Shared test setup.

Markers: ``gpu`` marks tests that run HIP kernels (they need a ROCm GPU and
libmoe355.so); everything else runs on the CPU. GPU tests call the product
through its C ABI / Python host code and check it against the CPU oracle in
oracle/ (fp64 restatement of the reference) on the same seeded inputs.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libmoe355.so")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")
