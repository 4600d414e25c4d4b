"""The reference-side binding (project-k3x_amd/host/binding/backend_hip.cpp)
compiles against the reference's own runtime/include: every pure virtual of
k3x::ComputeBackend (runtime/include/k3x/backend.hpp:326-462) is overridden
with the reference's exact signature (the factory instantiates the class, so
an abstract or mismatched one fails to build).  Linked with the reference's
CPU backend sources, it keeps the reference's error contract: only a shape
the library declines before any device work runs on make_cpu_backend() (and
is counted); a device failure is returned as a failure.  CPU only; skipped
where the reference tree is absent (the GPU box)."""
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


REF_SRC = "/root/reference/runtime/src"
DRIVER = os.path.join(ROOT, "tests", "cpp", "binding_fallback_driver.cpp")
PKG = os.path.join(ROOT, "project-k3x_amd")


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="reference tree absent")
@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
def test_binding_falls_back_only_on_declined_shapes():
    lib = os.path.join(PKG, "libk3x_hip_backend.so")
    assert os.path.exists(lib), "libk3x_hip_backend.so not built (__graft_entry__.build())"
    srcs = [os.path.join(REF_SRC, f) for f in ("backend_cpu.cpp", "ops.cpp", "routing_policy.cpp",
                                                  "expert_major.cpp", "official_moe.cpp",
                                                  "profile.cpp")]
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "binding_fallback")
        r = subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Wextra", f"-I{REF_INCLUDE}",
                            f"-I{os.path.join(PKG, 'host')}", "-o", exe, DRIVER, SRC, *srcs,
                            f"-L{PKG}", "-lk3x_hip_backend", f"-Wl,-rpath,{PKG}"],
                           capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stderr[-4000:]
        run = subprocess.run([exe], capture_output=True, text=True, timeout=120)
        assert run.returncode == 0, (run.returncode, run.stdout)
        assert run.stdout.count(": ok") == 4, run.stdout
