import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs on the GPU box only")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def hip():
    """The registered HIP backend for device 0 (GPU tests only)."""
    import oxmera_amd as ox
    n = ox.init()
    assert n >= 1, "no HIP device visible: GPU tests need the MI355X box"
    return ox.backend_for(ox.Device.rocm(0))
