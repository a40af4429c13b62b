import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


@pytest.fixture(scope="session")
def ctx():
    """One wgb_ctx on device 0 for the whole GPU session."""
    from wgblas_amd import Context, device_count

    if device_count() == 0:
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    c = Context(0)
    yield c
    c.close()
