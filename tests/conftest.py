import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built liblq.so")
    config.addinivalue_line("markers", "slow: longer CPU test")


def pytest_collection_modifyitems(config, items):
    """GPU tests are skipped only where there is no GPU at all; on a GPU box a missing liblq.so fails them."""
    try:
        import torch
        has_gpu = torch.cuda.device_count() > 0
    except Exception:
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this container")
    for it in items:
        if it.get_closest_marker("gpu") is not None:
            it.add_marker(skip)


@pytest.fixture(autouse=True)
def _announce(request):
    # GPU tests run in one process on the GPU box; print the case name before each so a fault names its test.
    if request.node.get_closest_marker("gpu") is not None:
        print("\n[gpu-case] %s" % request.node.nodeid, flush=True)
    yield
