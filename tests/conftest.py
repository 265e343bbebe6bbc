import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def dext():
    from moe_fused_inference_amd import get_decode_ext
    return get_decode_ext()


@pytest.fixture(scope="session")
def lext():
    from moe_fused_inference_amd import get_ext
    return get_ext()
