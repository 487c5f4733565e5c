import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "talking-portrait.cpp_amd")
for p in (ROOT, PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def om():
    from oracle import mdec
    mdec.lib()
    return mdec


@pytest.fixture(scope="session")
def oracle_fmt():
    from oracle import fmt, mdec
    mdec.lib()
    return fmt


@pytest.fixture(scope="session")
def oracle_menc():
    from oracle import mdec, menc
    mdec.lib()
    return menc


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a HIP device")
    return torch
