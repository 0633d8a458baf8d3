import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) and the built libimie_gfx950.so")


@pytest.fixture(scope="session")
def gpu():
    """The gpu_native module, asserting the device is really there (GPU tests never pass on a fallback)."""
    from integer_inference_engine_amd import gpu_native
    assert gpu_native.gpu_available(), "gpu-marked test without a usable gfx950 device"
    return gpu_native
