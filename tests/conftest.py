import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tensor-adapt_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(autouse=True)
def _release_device_tensors(request):
    """Drop the device tensors a GPU test made, after the device is idle."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import gpu_util
    import torch
    torch.cuda.synchronize()
    gpu_util.LIVE.clear()
