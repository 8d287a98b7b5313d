import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mobile-moe.zig_amd")
for p in (os.path.join(PKG, "python"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

# Present in the build container only; tests that read it skip elsewhere.
REFERENCE_SRC = "/root/reference/src"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; runs through the C ABI")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def mm():
    import mmhip
    return mmhip


@pytest.fixture(scope="session")
def ctx(mm):
    """A device context. On a GPU run a missing device is a failure, not a skip."""
    lib = mm.load_library()
    if not lib.mmhip_is_available():
        pytest.fail("no gfx950 device visible to libmmhip")
    c = mm.Context(0)
    yield c
    c.close()
