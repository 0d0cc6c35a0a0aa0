import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "x0ne-engine_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950); run with -m gpu on the GPU box")
    config.addinivalue_line("markers", "slow: a CPU test that takes more than a few seconds")


@pytest.fixture(scope="session")
def kernels():
    from x0ne_core.ops import Kernels
    return Kernels()
