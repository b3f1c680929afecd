import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests need both the card and libmaskahead_hip.so."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this host")
    from maskahead_amd import _native

    _native.load()          # raises if the library was not built: never a silent fallback
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before any GPU work, so a fault still leaves the test name behind
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield
