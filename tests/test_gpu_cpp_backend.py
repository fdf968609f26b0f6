"""Runs the C++23 HIPBackend caller (tests/cpp/test_hip_backend.cpp), which
exercises om::HIPBackend the way the reference's own GTest cases exercise
CPUBackend, including the throw-on-error contract."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "omnimatchdeeplearningtool_amd", "_build", "test_hip_backend")


def test_cpp_hip_backend():
    assert os.path.exists(EXE), "build the package first (python -m omnimatchdeeplearningtool_amd.build)"
    r = subprocess.run([EXE], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert "ALL PASSED" in r.stdout
