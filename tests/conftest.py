"""Shared test setup: import paths, the `gpu` marker, seeded fixtures.

Tests marked `gpu` need an MI355X and the built HIP library; everything else
runs on the CPU. The package directory (`grouped-nf4-gemm_amd/`, the analogue
of the reference's `kernel/`) and the repository root (for the `oracle`
test package) go on sys.path, so tests import `nf4_grouped` the way the
reference's tests do.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "grouped-nf4-gemm_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before any GPU work so a crash log says which test ran
    if "gpu" in request.keywords:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield
