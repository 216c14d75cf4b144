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


def pytest_terminal_summary(terminalreporter):
    """One line on the logits checks of this run: how close the GPU came to
    the reference order, and whether any row used the exception cap."""
    gu = sys.modules.get("gpu_util")
    rec = getattr(gu, "LOGITS_RECORD", None)
    if not rec:
        return
    worst = max(rec, key=lambda r: r[1])
    n_exc = sum(r[2] for r in rec)
    terminalreporter.write_line(
        f"logits checks: {len(rec)} calls, {sum(r[3] for r in rec)} rows; largest per-row "
        f"gpu-oracle L2 {worst[1]:.3e} ({worst[0]}); exception rows above 1e-2: {n_exc}")
