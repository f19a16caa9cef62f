"""Test configuration: the `gpu` marker (tests that launch HIP kernels on a
real MI355X) and shared helpers. CPU runs: `pytest -m "not gpu"`."""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built libpdhip.so")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _name_the_case(request):
    # print the case before it runs, so a GPU fault's output names it
    if "gpu" in request.node.keywords:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
