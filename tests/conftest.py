import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvvllm_hip.so on the device)")


@pytest.fixture(scope="session")
def oracle():
    """The CPU oracle (test infrastructure), built on first use."""
    from oracle import oracle as O
    if not O.available("port"):
        O.build(ref=True)
    return O


@pytest.fixture(scope="session")
def gpu():
    """Initialised C ABI on device 0 (GPU tests only)."""
    from vvllm_amd import capi
    capi.load()
    name = capi.init(0)
    print(f"[gpu] {name}", flush=True)
    yield capi
    capi.set_kernel(capi.KERNEL_AUTO)
    capi.sync()
