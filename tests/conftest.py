"""Shared pytest configuration.

Markers:
  gpu -- needs an MI355X (gfx950) and runs the HIP kernels through the C ABI.
Everything else runs on the CPU: the oracle against the reference's known
answers and closed forms, host utilities, and the C ABI's exports.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP kernels via the C ABI)")


@pytest.fixture(scope="session")
def rt():
    """The device-0 runtime.  GPU tests fail (not skip) if it cannot be created."""
    import ammon_amd

    runtime = ammon_amd.Runtime(0)
    yield runtime
    runtime.close()
