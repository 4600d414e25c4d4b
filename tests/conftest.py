"""pytest configuration: the `gpu` marker and import paths.

GPU tests (marked `gpu`) call the HIP library through its C ABI; everything
else runs on the CPU against the oracle and golden fixtures.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "project-k3x_amd", "tests"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X and the built HIP library")


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
