import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "dial-27b_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def O():
    import oracle as _o  # oracle/oracle.py -- the checker
    _o.build()
    return _o


@pytest.fixture(scope="session")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def dq():
    import dialq as _dq
    return _dq
