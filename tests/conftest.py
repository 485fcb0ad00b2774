"""Shared test setup.

- ``gpu`` marks tests that need an MI355X (run with ``-m gpu``); without a visible GPU
  they are skipped, never rerouted to a CPU path.
- ``pkg(name)`` imports a module of the product package, whose directory name
  (``oxr-inference_amd``) is not a Python identifier.
"""

from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PACKAGE = "oxr-inference_amd"


def pkg(name: str | None = None):
    return importlib.import_module(PACKAGE if name is None else f"{PACKAGE}.{name}")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built gfx950 library")


def pytest_collection_modifyitems(config, items):
    gpu_items = [item for item in items if "gpu" in item.keywords]
    if not gpu_items:
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in gpu_items:
        item.add_marker(skip)


def announce(*parts) -> None:
    """Print and flush what names the case before a GPU step."""
    print("[case]", *parts, flush=True)
