import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "rl-triton_amd"), ROOT, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long-running parity sizes")


@pytest.fixture(autouse=True)
def set_correctness_warnings(request):
    """Enable the reference's expensive input assertions for every test, as the
    reference's own conftest does (tests/conftest.py:12-24)."""
    old = os.environ.get("RL_TRITON_CORRECTNESS_WARNINGS")
    os.environ["RL_TRITON_CORRECTNESS_WARNINGS"] = "1"
    yield
    if old is None:
        del os.environ["RL_TRITON_CORRECTNESS_WARNINGS"]
    else:
        os.environ["RL_TRITON_CORRECTNESS_WARNINGS"] = old


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
