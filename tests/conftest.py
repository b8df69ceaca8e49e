import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def gpu_device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """Per-tensor parity errors of the GPU tests (max error / worst ratio to the bound)."""
    try:
        from tests.tolerance import SUMMARY
    except ImportError:
        from tolerance import SUMMARY  # tests/ on sys.path
    if SUMMARY:
        terminalreporter.write_sep("-", "parity: max abs error / worst ratio to the bound")
        for line in SUMMARY:
            terminalreporter.write_line(line)
