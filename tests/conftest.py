import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and libexq_hip.so")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def device():
    import torch
    return torch.device("cuda", 0)


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """One line per parity check: the errors the path's bound is stated on
    (relative L2 over the output, worst token row, max |y - ref|, and the
    reference's max|d|/rms(ref), scripts/bench_int4.py:88-91)."""
    try:
        from tests._helpers import PARITY_LOG
    except Exception:
        return
    if not PARITY_LOG:
        return
    tr = terminalreporter
    tr.write_sep("-", f"parity errors ({len(PARITY_LOG)} checks)")
    worst = max(PARITY_LOG, key=lambda r: r[1])
    for what, err, rerr, mx, mor in PARITY_LOG:
        tr.write_line(f"{what}: rel_l2={err:.3e} row={rerr:.3e} max_abs={mx:.3e} max/rms={mor:.3e}")
    tr.write_line(f"worst rel_l2 {worst[1]:.3e} ({worst[0]})")
