"""Test setup: import paths, the `gpu` marker, and GPU skip when no device is present.

`-m "not gpu"` runs everything that needs no GPU (oracle pins, host logic, C-ABI loading
and argument checks); `-m gpu` runs the parity tests that call the HIP library.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "vllm-expert-cache_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built library")


def pytest_collection_modifyitems(config, items):
    gpu_items = [it for it in items if "gpu" in it.keywords]
    if not gpu_items:
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for it in gpu_items:
        it.add_marker(skip)
