import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rakkan-mesh_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and librkhip.so")
    # The oracle is plain C; build it if this checkout has not yet.
    if not os.path.exists(os.path.join(ROOT, "oracle", "_build", "librkoracle.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


@pytest.fixture(scope="session")
def dev():
    import rkhip

    d = rkhip.Device(0)
    yield d
    d.close()
