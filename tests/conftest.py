import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def nncl():
    import torch
    from my_pytchon_opencl_lib_amd import NnClGlob
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return NnClGlob("cuda:0")


POLICIES = {"auto": 0, "tiled": 1, "small": 2, "skinny": 3, "panel": 4, "tiny": 5}


@pytest.fixture(params=sorted(POLICIES))
def policy(request):
    """Runs a test once per kernel family (migemm_set_gemm_policy), restoring AUTO after."""
    from my_pytchon_opencl_lib_amd import _native
    prev = _native.set_gemm_policy(POLICIES[request.param])
    yield request.param
    _native.set_gemm_policy(prev)
