import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# Error figures the parity tests measured ("cfg1 vs fp32 SDPA max ... mean ..."), printed after the run so a
# quiet (-q) run still shows them.
FIGURES = []


def record(line):
    """Keep one measured-figure line for the end-of-run summary (and print it for -s runs)."""
    FIGURES.append(line)
    print(line, flush=True)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    if FIGURES:
        terminalreporter.section("measured figures")
        for line in FIGURES:
            terminalreporter.write_line(line)


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def lib():
    from lingbot_world_v2_realtime_amd import _lib
    return _lib.load()
