"""Runs tests/cpp/ceilings.hip on cuda:0: the MFMA-only, LDS-fed MFMA and
x-staging-only ceilings of the tiled matmul's M = 2048 configuration, and the
compute ceilings of its dequant to bf16 tiles against the exact-codes
alternative (dequant applied to the accumulators), whose figures the design
notes quote.  Checks that it runs and that each figure is
in a physically possible range (below MI355X's dense bf16 peak and HBM
bandwidth scaled by the x re-reads it measures)."""
import os
import re
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "ceilings")


def test_ceilings(gpu):
    assert os.path.exists(BIN), f"{BIN} not built (make -C tests/cpp)"
    r = subprocess.run([BIN, "1024"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and "PASSED" in r.stdout, r.stdout + r.stderr
    tf = [float(v) for v in re.findall(r"([0-9.]+) TFLOP/s", r.stdout)]
    assert len(tf) == 4 and all(0 < v < 2600 for v in tf), tf
    gbs = [float(v) for v in re.findall(r"([0-9.]+) GB/s", r.stdout)]
    assert len(gbs) == 1 and gbs[0] > 0, gbs
