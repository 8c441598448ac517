import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PACKAGE = os.path.join(ROOT, "jade-compute_amd")
for path in (PACKAGE, os.path.dirname(os.path.abspath(__file__))):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def runtime():
    import jade_hip

    rt = jade_hip.HipRuntime(0)
    yield rt
    rt.close()


@pytest.fixture(scope="session")
def oracle():
    import oracle_binding

    return oracle_binding
