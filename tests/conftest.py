"""Shared pytest setup: the `gpu` marker, repo-root imports, device helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through libomhip.so)")


@pytest.fixture(scope="session")
def hip():
    """The loaded libomhip module, initialised on device 0 (GPU tests only)."""
    import omnimatchdeeplearningtool_amd as om
    om.init(0)
    name = om.device_name(0)
    print(f"\n[omhip] device 0: {name}", flush=True)
    return om


def to_dev(om, a):
    return om.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def empty_dev(om, shape, dtype=np.float32):
    return om.DeviceBuffer.empty(tuple(shape), dtype)
