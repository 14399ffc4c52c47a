"""pytest configuration: the `gpu` marker and import paths.

GPU tests are marked ``@pytest.mark.gpu`` (as in the reference's
tests/conftest.py:15-31) and are skipped when no GPU is visible; everything
else runs on the CPU.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "reflex-infer_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "host_path: exercises the host GEMV on purpose")


@pytest.fixture(autouse=True)
def _gpu_tests_compute_on_the_gpu(request):
    """A GPU test must not pass through the host GEMV (the C++ API's path for
    weights the GPU cannot read) unless it is marked host_path."""
    if "gpu" not in request.keywords or "host_path" in request.keywords:
        yield
        return
    try:
        from rxq4 import capi
        before = capi.host_gemv_calls()
    except Exception:
        yield
        return
    yield
    assert capi.host_gemv_calls() == before, "a GPU test computed through the host GEMV"


def pytest_collection_modifyitems(config, items):
    if any("gpu" in item.keywords for item in items) and not _gpu_available():
        skip = pytest.mark.skip(reason="no GPU visible")
        for item in items:
            if "gpu" in item.keywords:
                item.add_marker(skip)
