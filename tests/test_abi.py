"""The C ABI library: it loads, exports every entry point include/*.h declares,
its ctypes declarations cover exactly those, and the host-side argument
checks fail closed with the documented status codes.  No device work: these
run without a GPU."""
from __future__ import annotations

import ctypes as C
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(k3x_hip_\w+)\s*\(", text):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    import k3x_amd
    return k3x_amd.load()


def test_headers_exist():
    assert HEADERS, "include/*.h missing"


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_declarations():
    import k3x_amd
    assert set(k3x_amd.EXPORTED) == declared_functions()


def test_status_names(lib):
    # error_code_name (runtime/include/k3x/status.hpp:33-56)
    assert lib.k3x_hip_status_name(0) == b"OK"
    assert lib.k3x_hip_status_name(9) == b"INVALID_EXTENT"
    assert lib.k3x_hip_status_name(14) == b"TENSOR_NOT_FOUND"
    assert lib.k3x_hip_status_name(15) == b"INVALID_MXFP4"
    assert lib.k3x_hip_status_name(16) == b"INVALID_STATE"
    assert lib.k3x_hip_status_name(17) == b"BACKEND_UNAVAILABLE"


def test_null_handles_fail_closed(lib):
    import k3x_amd
    assert lib.k3x_hip_ctx_destroy(None) == k3x_amd.ERR_INVALID_EXTENT
    assert lib.k3x_hip_ctx_synchronize(None) == k3x_amd.ERR_INVALID_EXTENT
    assert lib.k3x_hip_ctx_set_profiling(None, 1) == k3x_amd.ERR_INVALID_EXTENT
    assert lib.k3x_hip_bank_destroy(None) == k3x_amd.ERR_INVALID_EXTENT
    assert lib.k3x_hip_bank_bytes(None) == 0
    assert lib.k3x_hip_ctx_create(0, None) == k3x_amd.ERR_INVALID_EXTENT
    p = k3x_amd.make_params(2, 16)
    assert lib.k3x_hip_moe_forward(None, None, C.byref(p), None, None, None) == \
        k3x_amd.ERR_INVALID_EXTENT


def test_context_without_device_is_unavailable(lib):
    """On a host without a visible GPU the context reports backend_unavailable
    (the reference's CUDA stub contract, runtime/src/backend_cuda_stub.cpp:6-10)."""
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    import k3x_amd
    h = C.c_void_p()
    assert lib.k3x_hip_ctx_create(0, C.byref(h)) == k3x_amd.ERR_BACKEND_UNAVAILABLE
    assert not h.value


def test_python_context_refuses_without_gpu():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    import k3x_amd
    with pytest.raises(RuntimeError):
        k3x_amd.Context(0)
