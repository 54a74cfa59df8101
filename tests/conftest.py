"""Shared pytest setup: repo root on sys.path and the `gpu` marker.

Tests marked `gpu` need an MI355X (gfx950) and the built HIP library; every
other test runs on the CPU (oracle, host logic, library load/exports).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X and the built HIP library")


def gpu_present() -> bool:
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def hip():
    """The product backend (C ABI over libmlk_hip.so), GPU tests only."""
    from mlk2_amd import backend
    be = backend.HipBackend()
    if not be.device_available():
        pytest.fail("gpu test run without a usable HIP device (libmlk_hip reports none)")
    return be
