"""Shared pytest configuration.

Markers: ``gpu`` -- needs an MI355X (run with ``-m gpu``); everything else runs
on the CPU and never launches a kernel.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def _gpu_ready() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail (not skip) if the HIP library is absent."""
    if not _gpu_ready():
        pytest.skip("no GPU visible")
    from spikeinfer_amd import _lib

    _lib.load()  # raises KernelLibraryMissing when the .so was not built
    import torch

    return torch.device("cuda:0")
