"""Runs the C++ host-layer test (tests/cpp/test_host_api.cpp) on cuda:0
against the C oracle: QuantizedLinear with and without bias, gather_qmm /
SwitchLinear (shared and per-selection x, grouped workspace),
QuantizedEmbedding, the Checkpoint reader on a small MLX model directory
written here, and the exception paths of include/miqmm.hpp."""
import os
import subprocess

import pytest

from test_checkpoint import QUANT, make_model

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "test_host_api")


def test_cpp_host_api(gpu, tmp_path):
    assert os.path.exists(BIN), f"{BIN} not built (make -C tests/cpp)"
    make_model(str(tmp_path), QUANT, shards=2)
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and "PASSED" in r.stdout, r.stdout + r.stderr
    for name in ("embed_tokens: QuantizedEmbedding", "q_proj: QuantizedLinear", "down_proj: QuantizedLinear",
                 "gate_proj: SwitchLinear", "SwitchLinear grouped x", "SwitchLinear grouped GEMV"):
        assert any(line.startswith("ok") and name in line for line in r.stdout.splitlines()), name
