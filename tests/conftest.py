import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def ctx():
    """One context for the GPU session. Fails (does not skip) when the native build or the device
    is missing: a GPU test must never pass on a fallback."""
    from moearc_amd import Context
    c = Context()
    print(f"\n[moearc] device: {c.device_name()}", flush=True)
    yield c
    c.close()
