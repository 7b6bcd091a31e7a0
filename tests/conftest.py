import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "htp-ops-lib-sd.cpp_amd")
ORACLE = os.path.join(REPO, "oracle")
GOLDEN = os.path.join(REPO, "tests", "golden")
for p in (PKG, ORACLE, GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def hip():
    """The library, initialised on GPU 0.  Fails (never skips) when the GPU
    path cannot be used, so a GPU run cannot pass without native code."""
    import htp_ops

    htp_ops.init(0)
    return htp_ops


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle
