import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


def pytest_collection_modifyitems(config, items):
    gpu_items = [item for item in items if "gpu" in item.keywords]
    if not gpu_items:
        return
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this container")
    for item in gpu_items:
        item.add_marker(skip)


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the test on stdout before it runs, so a GPU run that dies names its case.
    if "gpu" in request.keywords:
        print(f"\n[gpu-test] {request.node.nodeid}", flush=True)
    yield
