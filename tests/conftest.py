import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs through the C-ABI")


@pytest.fixture(scope="session")
def native():
    """The product library (raises if it is not built: there is no fallback)."""
    import cudaforge_amd
    return cudaforge_amd.load_library()


@pytest.fixture(scope="session")
def gpu(native):
    """Initialise device 0; fails loudly if no HIP device is present."""
    import cudaforge_amd
    if not cudaforge_amd.gpu_available():
        pytest.fail("no HIP device visible: GPU tests must run on the MI355X box")
    cudaforge_amd.init_gpu(0)
    return native
