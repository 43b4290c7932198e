import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "loomformer-paraplex_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# measured errors recorded by tests (name -> value), printed in the run's
# terminal summary so that they stay in the log whatever the capture mode
_MEASURED = []


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


@pytest.fixture(scope="session")
def golden_dir():
    return os.path.join(ROOT, "tests", "golden")


@pytest.fixture
def measured(request):
    """measured(name, value): keep a measured figure for the run's summary."""
    def rec(name, value):
        _MEASURED.append((request.node.nodeid, name, value))
        print(f"[measured] {name} = {value}", flush=True)
    return rec


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    if not _MEASURED:
        return
    terminalreporter.section("measured errors")
    for nodeid, name, value in _MEASURED:
        v = f"{value:.3e}" if isinstance(value, float) else str(value)
        terminalreporter.write_line(f"{nodeid}: {name} = {v}")
