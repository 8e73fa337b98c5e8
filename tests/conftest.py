import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    """Order GPU tests so that a test file named test_zz_* runs last."""
    items.sort(key=lambda item: 1 if os.path.basename(str(item.fspath)).startswith("test_zz_") else 0)


@pytest.fixture(scope="session")
def golden():
    from tests.golden_util import Golden
    return Golden()
