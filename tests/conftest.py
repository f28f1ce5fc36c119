import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def gpu():
    """The HIP product library bound to device 0.  Fails loudly (no CPU
    fallback) when the extension or the GPU is missing."""
    from fe2o3_amd import runtime
    ctx = runtime.GpuContext.current()
    yield ctx
    ctx.synchronize()
