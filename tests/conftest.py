import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on the device)")
    config.addinivalue_line("markers", "slow: long CPU-only checks (opt-in with CZ_SLOW=1)")


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import oracle as orc
    orc.build()
    return orc


@pytest.fixture(scope="session")
def gpu():
    """Initialises the HIP library on cuda:0; fails (does not skip) when the
    library is missing or no device answers - GPU tests never fall back."""
    from colizig_amd import moe
    name = moe.init()
    assert "gfx950" in name, name
    yield name
