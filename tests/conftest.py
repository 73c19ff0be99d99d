import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "glm-5.3-kernels_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on CPU")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)
    return torch.device("cuda:0")


def log_case(*parts):
    """Print (and flush) what names the case before a GPU step."""
    print("[case]", *parts, flush=True)


def pytest_terminal_summary(terminalreporter):
    """The parity magnitudes the GPU tests recorded (parity_log), after the
    test results, so that the end of the run's output carries them."""
    import parity_log
    lines = parity_log.summary_lines()
    if lines:
        terminalreporter.write_sep("-", "parity against the oracle")
        for line in lines:
            terminalreporter.write_line(line)
