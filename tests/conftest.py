import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the HIP product")


@pytest.fixture(scope="session", autouse=True)
def _oracle_threads():
    """The checker's row loops on all host cores (at most 16); its results do
    not depend on the thread count."""
    import pyoracle as po
    try:
        po.set_threads(po.default_threads())
    except ImportError:
        pass  # oracle not built: the tests that need it fail on their own
    yield


@pytest.fixture(scope="session")
def gpu():
    """torch on the HIP device; GPU tests fail loudly when none is visible."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    return torch.device("cuda:0")
