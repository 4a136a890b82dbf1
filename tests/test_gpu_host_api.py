"""Runs the C++ host-layer test (tests/cpp/test_host_api.cpp): QuantizedLinear
with and without bias, and the exception path of include/miqmm.hpp, on cuda:0
against the C oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "test_host_api")


def test_cpp_host_api(gpu):
    assert os.path.exists(BIN), f"{BIN} not built (make -C tests/cpp)"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and "PASSED" in r.stdout, r.stdout + r.stderr
