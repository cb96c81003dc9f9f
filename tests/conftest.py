import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "encoding-experiment_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through liblarql_hip on cuda:0)")


@pytest.fixture(scope="session")
def hip():
    """One HIP backend context for the whole GPU session."""
    import larql_hip

    be = larql_hip.HipBackend(0, strict=True)
    print(f"[hip] {be.device_info()}", flush=True)
    yield be
    be.close()
