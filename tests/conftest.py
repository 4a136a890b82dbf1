import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "sen-mlx_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmiqmm.so on cuda:0)")


@pytest.fixture(scope="session")
def c_oracle():
    import oracle as O

    O.build_c_oracle()
    return O


@pytest.fixture(scope="session")
def gpu():
    """torch on cuda:0 with libmiqmm.so loaded; skips without a GPU, fails if the library is missing"""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import miqmm

    miqmm.lib()  # raises if libmiqmm.so is not built
    return torch.device("cuda:0")
