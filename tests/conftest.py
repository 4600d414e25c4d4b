"""pytest configuration: the `gpu` marker, import paths and the parity report.

GPU tests (marked `gpu`) call the HIP library through its C ABI; everything
else runs on the CPU against the oracle and golden fixtures.  Tests record
the figures their checks rest on (fractions within tolerance, worst ulps)
with the `parity_report` fixture; they are printed in a section of the
terminal summary, which also appears under `pytest -q`.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "project-k3x_amd", "tests"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)

_REPORT: list[str] = []


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X and the built HIP library")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    if _REPORT:
        terminalreporter.section("parity report")
        for line in _REPORT:
            terminalreporter.write_line(line)


@pytest.fixture
def parity_report(request):
    """parity_report(text): one line of the terminal summary, prefixed with
    the test's id."""
    def add(text: str) -> None:
        _REPORT.append(f"{request.node.nodeid}: {text}")
    return add


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reflib():
    from oracle import REF_SO, RefLib
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref/libk3x_ref.so not built (needs the reference tree)")
    return RefLib()
