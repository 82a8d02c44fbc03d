import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "webgpu-gemma_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libgg.so")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    """The oracle library travels prebuilt; build it here when it is absent."""
    from oracle import oracle as orc
    if not os.path.exists(orc.LIB_PATH):
        from oracle import build
        build.build_oracle()
    yield


@pytest.fixture(scope="session")
def gpu():
    """Device handle for GPU tests; fails loudly when the HIP path is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    from gemma_amd import capi
    capi.lib()  # raises if libgg.so was not built
    return torch.device("cuda:0")
