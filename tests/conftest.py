import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (built from oracle/ if needed)."""
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def rvlib():
    """librvmoe.so, built in-tree when it is missing (no GPU needed to load it)."""
    from rosevine_amd import build, hip
    if not os.path.exists(hip.LIB_PATH):
        build.build()
    return hip.lib()


@pytest.fixture(scope="session")
def gpu(rvlib):
    """The HIP device, initialised once for the GPU tests."""
    from rosevine_amd import hip
    print(f"[gpu] init device 0", flush=True)
    hip.init(0)
    return hip
