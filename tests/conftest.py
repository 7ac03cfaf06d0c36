import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mimo-on-a-mac_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libmimo_moe.so")


@pytest.fixture
def rng():
    """A fresh seeded generator per test: a test's inputs do not depend on which tests ran before it."""
    import numpy as np
    return np.random.default_rng(0)
