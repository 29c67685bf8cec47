import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def K():
    import kuiperllama_amd

    return kuiperllama_amd


@pytest.fixture(scope="session")
def O():
    import oracle

    return oracle


@pytest.fixture(scope="session")
def gpu(K):
    """The GPU tests run only where a device is present; on a GPU box a
    missing or broken native library is an error, never a skip."""
    n = K.device_count()
    if n < 1:
        pytest.fail("no HIP device visible to a test marked gpu")
    return n
