"""Shared fixtures.  ``-m gpu`` tests need a ROCm GPU and the built
libortho_amd.so; the rest run on the CPU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libortho_amd.so")


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from libortho_amd import _lib
    _lib.lib()  # fails loudly if the HIP library is missing
    return torch.device("cuda:0")
