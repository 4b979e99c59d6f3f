import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C ABI of libnibble_hip.so")


def _print_case(item):
    # Name the case before any GPU work starts, so a run that dies mid-test still says which one it was.
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu case] {item.nodeid}", flush=True)


def pytest_runtest_setup(item):
    _print_case(item)


@pytest.fixture(scope="session")
def backend():
    """One HipBackend on device 0 for the whole GPU session."""
    import nibble_amd

    be = nibble_amd.HipBackend(0)
    yield be
    be.close()
