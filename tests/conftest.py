"""Shared test setup.

Markers: `gpu` = needs an MI355X (HIP kernels through libnanoserve_hip.so). On a machine without a GPU those
tests skip; on a GPU machine the library must load (no silent fallback), or the session errors.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="needs a GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def hiplib():
    """The loaded kernel library (GPU tests only): raises if it is missing."""
    from nanoserve_amd import _lib
    return _lib.load_library()


def cpu_gen(seed: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(seed)
