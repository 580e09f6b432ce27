"""Shared test setup.

Markers: `gpu` tests need an MI355X and call the HIP path through the C ABI;
everything else runs on the CPU (oracle checks, host logic, ABI surface).
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; calls libcleave_hip.so kernels")


@pytest.fixture(scope="session")
def golden():
    return json.loads((ROOT / "tests" / "golden" / "reference_vectors.json").read_text())


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def hip():
    """The product library on a real device.  A missing library or device is an
    error here, never a skip: GPU tests only run where a GPU is expected."""
    import cleave_amd as ca
    assert ca.device_available(), "no HIP device visible to libcleave_hip.so"
    ca.init()
    return ca
