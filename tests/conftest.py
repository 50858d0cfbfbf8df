import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "tablemoe-sc26_amd"
for p in (str(REPO), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def hip_device():
    """The HIP device for parity tests.  GPU tests fail (never skip) without one."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a HIP device")
    from table_moe import _native

    _native.load()  # raise if the library is not built: no fallback path exists
    from table_moe.cache_engine import GlobalTable

    # every layer call of the GPU tests checks the workspace's error word: a
    # bounded cross-workgroup wait that ran out fails the test that made it
    GlobalTable.check_waits = True
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    return dev


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before any GPU work so a failing run says which one
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield


os.environ.setdefault("PYTHONHASHSEED", "0")
