"""Shared test setup.

Markers: ``gpu`` -- needs a real MI355X (run with ``-m gpu`` on the GPU box);
everything else runs on a CPU-only host.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X GPU (libenchip.so on cuda:0)")


@pytest.fixture(scope="session")
def ctx():
    """One enchip context for the GPU session. Fails loudly (no skip) when the
    library or the device is missing: a GPU test must never pass on a fallback."""
    from aikit_amd import enchip

    c = enchip.Context(0)
    info = c.device_info()
    print(f"\n[enchip] device {info}", flush=True)
    yield c
    c.close()


@pytest.fixture(scope="session")
def workers():
    """Host threads for the AVX2 CPU checker (the GPU box's CPU share is 16)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))
