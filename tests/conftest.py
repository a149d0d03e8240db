"""Shared pytest setup.

* Puts the package root (decode-kernel_amd/, like the reference's
  `pythonpath = ["python"]`, pyproject.toml:19-21) and the repo root (for
  oracle/) on sys.path.
* Registers the `gpu` marker. GPU tests are deselected with -m "not gpu"; if
  they are selected on a machine without a GPU they are skipped. On a GPU
  machine a missing extension is an error, never a skip.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "decode-kernel_amd"
for p in (str(PKG_ROOT), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP extension")


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        have_gpu = torch.cuda.is_available()
    except Exception:
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
