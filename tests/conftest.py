import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def kernels():
    import roost_amd

    return roost_amd.library()


@pytest.fixture(scope="session")
def session(kernels):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import roost_amd

    s = roost_amd.OpSession(kernels, device=0)
    yield s
    s.close()


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work so a run that dies mid-test still says which case it was.
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
