"""Test setup: make the package and the oracle importable without an install, register the
``gpu`` marker, and skip GPU tests cleanly when no HIP device is visible."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "pto-fuser_amd"))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:                       # pragma: no cover - torch missing
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def announce(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a box that dies still shows it)."""
    print(f"[gpu-case] {msg}", flush=True)
