"""The C++ host side (k3x_amd::HipMoeBackend, project-k3x_amd/host/): the
library loads and exports the factory and the ComputeBackend-shaped methods;
without a GPU the factory fails closed with backend_unavailable (the
reference's CUDA stub contract, runtime/src/backend_cuda_stub.cpp:6-10).
The GPU behaviour is tests/test_gpu_host_backend.py."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "project-k3x_amd", "libk3x_hip_backend.so")
EXE = os.path.join(ROOT, "tests", "cpp", "test_hip_backend")
METHODS = ["k3x_amd::make_hip_backend", "k3x_amd::HipMoeBackend::mxfp4_situ_mlp_group",
           "k3x_amd::HipMoeBackend::mxfp4_situ_mlp_batch",
           "k3x_amd::HipMoeBackend::mxfp4_situ_mlp_grid", "k3x_amd::HipMoeBackend::mxfp4_situ_moe",
           "k3x_amd::HipMoeBackend::mxfp4_situ_moe_tokens",
           "k3x_amd::HipMoeBackend::expert_major_block_moe",
           "k3x_amd::HipMoeBackend::official_mxfp4_moe_ffn",
           "k3x_amd::HipMoeBackend::official_mxfp4_moe_ffn_prepared",
           "k3x_amd::HipMoeBackend::prepare_official_moe_route",
           "k3x_amd::HipMoeBackend::discard_official_moe_prepared",
           "k3x_amd::HipMoeBackend::runtime_stats", "k3x_amd::error_code_name"]


def test_library_loads_and_exports_the_methods():
    assert os.path.exists(LIB), "libk3x_hip_backend.so not built (__graft_entry__.build())"
    C.CDLL(LIB)
    out = subprocess.run(["nm", "-DC", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    missing = [m for m in METHODS if m + "(" not in out]
    assert not missing, missing


def test_factory_fails_closed_without_a_device():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    assert os.path.exists(EXE), "tests/cpp/test_hip_backend not built (__graft_entry__.build())"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "BACKEND_UNAVAILABLE" in r.stdout, (r.returncode, r.stdout)


def test_host_checks_without_a_device():
    """Argument and shape contract on a backend with no device attached
    (tests/cpp/host_checks_driver.cpp): declined shapes are marked declined
    before any device work; a device failure is not; one tensor id for two
    tensors of a call is rejected before any upload."""
    exe = os.path.join(ROOT, "tests", "cpp", "host_checks_driver")
    assert os.path.exists(exe), "tests/cpp/host_checks_driver not built (__graft_entry__.build())"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, (r.returncode, r.stdout)
    assert r.stdout.count(": ok") == 4, r.stdout
