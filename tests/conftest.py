"""Shared pytest configuration.

* ``gpu`` marks tests that need an MI355X (run with ``-m gpu``); everything else
  runs on a CPU-only host (``-m "not gpu"``).
* The product package lives in ``flash-attention-legacy_amd/`` and the oracle in
  ``oracle/``; both are put on ``sys.path`` here.
* After every GPU test the device is synchronised so an asynchronous fault is
  reported against the test that caused it (as in the reference's
  tests/conftest.py:27-32).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "flash-attention-legacy_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (gfx950)")
    config.addinivalue_line("markers", "slow: long-running test")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _sync_after_gpu_test(request):
    yield
    if "gpu" in request.keywords and _gpu_available():
        import torch
        torch.cuda.synchronize()
