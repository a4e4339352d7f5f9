import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; runs through the C ABI")


@pytest.fixture(scope="session")
def rocm():
    """One HIP backend context for the GPU tests (loads fail loudly if the library is missing)."""
    from silvic_amd import RocmBackend

    if not RocmBackend.available():
        pytest.fail("no gfx950 device visible to the HIP runtime")
    b = RocmBackend()
    yield b
    b.close()
