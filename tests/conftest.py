"""Shared pytest setup.

Markers:
  gpu -- needs an MI355X (gfx950) and the built libcormorant_amd.so.  GPU tests
         are skipped only when no GPU device exists at all; on a GPU host a
         missing or unloadable library is a hard failure, never a fallback.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an MI355X GPU and the HIP library")


def _have_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _have_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU device present")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
