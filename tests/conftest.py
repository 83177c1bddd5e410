import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "verum-bespoke-singularity_amd")
for p in (PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs on the MI355X box)")
    config.addinivalue_line("markers", "slow: long-running CPU check")


@pytest.fixture(scope="session")
def oracle():
    from oracle_lib import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def host():
    import vbs_gfx950
    return vbs_gfx950.load_host()


@pytest.fixture(scope="session")
def dev():
    """The gfx950 device library, initialised. A GPU test fails (it does not
    skip) when the device cannot be opened."""
    import vbs_gfx950
    d = vbs_gfx950.DeviceLib()
    if not d.init():
        raise RuntimeError(f"gfx950 device unavailable: {d.error()}")
    return d


@pytest.fixture(scope="session")
def backend(dev):
    import vbs_gfx950
    b = vbs_gfx950.gfx950_backend()
    if not b.init():
        raise RuntimeError(f"g_vbs_hip_backend init failed: {b.last_error()}")
    return b
