import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")
    import helpers

    helpers.PYTEST_CONFIG = config


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O.build()
    return O


def gpu_ready() -> bool:
    try:
        from ferrisboost_amd import _native as N

        return N.device_available(0)
    except Exception:
        return False


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any device work so a failing GPU step is attributable.
    if request.node.get_closest_marker("gpu"):
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield
