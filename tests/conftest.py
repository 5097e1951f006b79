import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

# Load what is built; build only if nothing is.
__graft_entry__._ensure_built()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


@pytest.fixture(scope="session")
def ctx():
    import channel_amd as ca
    c = ca.Context(0)
    yield c
    c.close()
