"""Shared pytest configuration.

Markers: ``gpu`` tests need a ROCm device and the built HIP library; they are
skipped when no GPU is visible.  CPU tests cover the oracle, the host logic
and the C ABI surface.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) device and the HIP library")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def built_lib():
    """Path of the in-tree HIP library, building it if it is missing."""
    from moe_amd import _lib
    if not _lib.LIB_PATH.exists():
        from moe_amd import build
        build.build()
    return _lib.LIB_PATH
