import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libtgohip.so")


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("a gpu-marked test ran without a visible GPU")
    return torch


@pytest.fixture(scope="session")
def ctx(torch_gpu):
    """One library context for the session, launching on torch's current stream so
    torch-side allocations and the library's kernels are ordered."""
    import tgo_amd
    c = tgo_amd.Context(0)
    c.set_stream(torch_gpu.cuda.current_stream().cuda_stream)
    yield c
    c.close()


def pytest_sessionstart(session):
    """Build the product library and the oracle if nothing is built yet (a fresh checkout);
    an existing build is used as it is."""
    import tgo_amd
    if not os.path.exists(tgo_amd.LIB_PATH):
        from tgo_amd import build
        build.build()
