import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; skips only when this machine has no GPU at all (never hides a missing
    library on a GPU machine: the kernels' loader raises in that case)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    return torch.device("cuda:0")


@pytest.fixture
def diag():
    """The library's diagnostic switches for one test (LQ_MX_REQUIRE_ROWS, ...): .set(names)
    turns switches on, .clear(names) off; the test's end restores the previous set."""
    from layer_quant_amd import _abi

    prev = _abi.diagnostics()

    class Switches:
        @staticmethod
        def set(*names):
            _abi.set_diagnostics(_abi.diagnostics() | set(names))

        @staticmethod
        def clear(*names):
            _abi.set_diagnostics(_abi.diagnostics() - set(names))

    yield Switches()
    _abi.set_diagnostics(prev)


def pytest_runtest_setup(item):
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {item.nodeid}", flush=True)


def pytest_terminal_summary(terminalreporter):
    """Measurements that GPU tests register in helpers.REPORT (e.g. the config-4 drift table),
    printed after the run so that they appear next to the final result line."""
    import helpers

    if helpers.REPORT:
        terminalreporter.section("measurements")
        for line in helpers.REPORT:
            terminalreporter.write_line(line)
