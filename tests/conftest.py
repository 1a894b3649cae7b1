"""Shared pytest configuration.

Markers: ``gpu`` — needs a ROCm device and libhimuon_hip.so (run with
``-m gpu`` on an MI355X); everything else runs on the CPU.
"""

from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires a ROCm GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running test")


@pytest.fixture(autouse=True)
def _gpu_cleanup_between_tests():
    """Drain the device between tests (allocator state must not leak across
    tests; mirrors the reference's tests/conftest.py:16-31)."""
    yield
    if torch.cuda.is_available():
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
