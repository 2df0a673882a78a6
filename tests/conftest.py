"""Shared pytest setup: the `gpu` marker, repo on sys.path, GPU helpers."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def config5_host():
    """BASELINE config 5 inputs (X [8192, 4096], W [14336, 4096], dY [8192,
    14336], bf16) from the CPU generator with seed 0: the tensors bench.py
    times."""
    import torch

    import bench

    return bench.config5_inputs(torch)


@pytest.fixture(scope="session")
def dev():
    import torch

    from practice_cuda_amd import _lib

    _lib.lib()  # fail loudly (not skip) when the HIP library is missing
    return torch.device("cuda:0")
