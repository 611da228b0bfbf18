import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from catfuse_amd import _hip
    _hip.lib()  # raises if the HIP library is not built
    return torch.device("cuda", 0)


def pytest_collection_modifyitems(config, items):
    # GPU tests print their node id first so a fatal GPU error names the case.
    for item in items:
        if item.get_closest_marker("gpu") is not None:
            item.user_properties.append(("gpu", True))


@pytest.fixture(autouse=True)
def _announce(request):
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
    yield
