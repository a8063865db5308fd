import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libdance_hip.so")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(autouse=True)
def _announce(request):
    # Names the case before any GPU work starts, so a box that dies mid-test
    # still leaves the test id in the log.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
