"""The reference-side binding (project-k3x_amd/host/binding/backend_hip.cpp)
compiles against the reference's own runtime/include: every pure virtual of
k3x::ComputeBackend (runtime/include/k3x/backend.hpp:326-462) is overridden
with the reference's exact signature (the factory instantiates the class, so
an abstract or mismatched one fails to build).  CPU only; skipped where the
reference tree is absent (the GPU box)."""
from __future__ import annotations

import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INCLUDE = "/root/reference/runtime/include"
SRC = os.path.join(ROOT, "project-k3x_amd", "host", "binding", "backend_hip.cpp")


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="reference tree absent")
@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
def test_binding_compiles_against_reference_headers():
    with tempfile.TemporaryDirectory() as d:
        obj = os.path.join(d, "backend_hip.o")
        r = subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Wextra", "-Werror", "-c",
                            f"-I{REF_INCLUDE}", f"-I{os.path.join(ROOT, 'project-k3x_amd', 'host')}",
                            SRC, "-o", obj], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-4000:]
        nm = subprocess.run(["nm", "-C", obj], capture_output=True, text=True, timeout=60)
        # The factory beside make_cuda_backend, defined here.
        assert "k3x::make_hip_backend(k3x::BackendOptions const&, k3x::Profiler*)" in nm.stdout
