import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "s2pro-native_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


@pytest.fixture(autouse=True)
def _keep_device_buffers_alive():
    """Device buffers created through gpu_util live until the test's GPU work
    has finished."""
    yield
    import gpu_util
    if gpu_util.LIVE:
        import torch
        torch.cuda.synchronize()
        gpu_util.LIVE.clear()
