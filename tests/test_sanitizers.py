"""Host code that parses untrusted input, built with AddressSanitizer and
UndefinedBehaviorSanitizer and run on the CPU (tests/cpp/sanitize_driver.cpp):

* the K3X reader's open-time checks (project-k3x_amd/csrc/k3x_reader.cpp) over
  the corrupted files of tests/test_storage.py and 300 seeded mutants of a
  good file (byte changes in the superblock, the directories and the payload,
  and truncations); every status must equal the library's own open; then the
  checksum verification (CRC32C, directory and root SHA-256) of every mutant
  that opens, which must equal the library's own k3x_hip_storage_verify;
* HipMoeBackend's argument checks (project-k3x_amd/host/k3x_hip_checks.hpp)
  over 20,000 randomised views: extents that disagree with their spans,
  products past SIZE_MAX, zero and odd sizes, 0xFF scales, non-finite values.

Any sanitizer report fails the test.  Skipped where g++ cannot build with the
sanitizers."""
from __future__ import annotations

import os
import struct
import subprocess

import numpy as np
import pytest

from test_storage import open_status, reader_cases

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER_SRC = os.path.join(ROOT, "tests", "cpp", "sanitize_driver.cpp")
READER_SRC = os.path.join(ROOT, "project-k3x_amd", "csrc", "k3x_reader.cpp")
FLAGS = ["-std=c++20", "-O1", "-g", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-Wall", "-Wextra",
         "-Werror", f"-I{os.path.join(ROOT, 'project-k3x_amd', 'host')}",
         f"-I{os.path.join(ROOT, 'project-k3x_amd', 'csrc')}", f"-I{os.path.join(ROOT, 'include')}"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("sanitize") / "sanitize_driver")
    r = subprocess.run(["g++", *FLAGS, DRIVER_SRC, READER_SRC, "-o", exe], capture_output=True,
                       text=True, timeout=300)
    if r.returncode != 0 and "sanitize" in r.stderr:
        pytest.skip("g++ without the sanitizer runtimes")
    assert r.returncode == 0, r.stderr[-4000:]
    return exe


def run(exe, *args):
    r = subprocess.run([exe, *args], capture_output=True, text=True, timeout=600, env=ENV)
    report = [m for m in ("AddressSanitizer", "LeakSanitizer", "runtime error:")
              if m in r.stderr]
    assert r.returncode == 0 and not report, r.stderr[-4000:]
    return r.stdout


def mutants(good: str, out_dir, n: int):
    data = open(good, "rb").read()
    rng = np.random.default_rng(11)
    paths = []
    for i in range(n):
        b = bytearray(data)
        kind = i % 4
        if kind == 0:  # superblock fields (the CRC then usually fails first)
            for _ in range(1 + i % 3):
                b[int(rng.integers(0, 4096))] = int(rng.integers(0, 256))
        elif kind == 1:  # directory bytes behind a valid superblock CRC
            at = int(rng.integers(4096, min(len(b), 4 * 4096)))
            b[at:at + 8] = struct.pack("<Q", int(rng.integers(0, 2**63)))
        elif kind == 2:  # truncation
            b = b[:int(rng.integers(0, len(b)))]
        else:  # payload bytes
            b[int(rng.integers(0, len(b)))] ^= 0xFF
        p = str(out_dir / f"mutant{i}.k3x")
        open(p, "wb").write(bytes(b))
        paths.append(p)
    return paths


def test_reader_under_sanitizers(driver, oracle, tmp_path):
    cases = reader_cases(oracle, tmp_path)
    paths = [p for p, _ in cases] + mutants(cases[0][0], tmp_path, 300)
    got = [int(v) for v in run(driver, "reader", *paths).split()]
    assert got[:len(cases)] == [want for _, want in cases]
    lib = [open_status(p) for p in paths]
    assert got == lib
    assert len(set(got)) >= 5  # the mutants reach several distinct checks


def test_backend_checks_under_sanitizers(driver):
    out = run(driver, "checks", "1", "20000")
    assert out.startswith("checks: 20000 views")


def test_reader_verification_under_sanitizers(driver, oracle, tmp_path):
    import k3x_amd
    cases = reader_cases(oracle, tmp_path)
    paths = [p for p, _ in cases] + mutants(cases[0][0], tmp_path, 120)
    got = [tuple(int(v) for v in line.split()) for line in
           run(driver, "verify", *paths).strip().splitlines()]
    assert got[0] == (0, 0)  # the good file opens and verifies
    opened = 0
    for path, (st, vst) in zip(paths, got):
        s = k3x_amd.Storage(path)
        assert s.open_status == st
        if st == 0:
            opened += 1
            assert s.verify() == vst, os.path.basename(path)
        s.close()
    # Payload mutants open and then fail their CRC: the verification runs.
    assert opened > 10 and any(v in (10, 11, 12, 13) for _, v in got)


def test_sha256_under_sanitizers(driver, tmp_path):
    """The reader's SHA-256 (FIPS 180-4, round constants derived at first
    use) against Python's hashlib: the FIPS 180-4 example messages ("abc", the
    448-bit two-block message, one million "a"), the empty message, every
    length around the 55/56/64-byte padding boundaries, and random lengths, each
    fed to the hash in pieces of several sizes."""
    import hashlib
    rng = np.random.default_rng(7)
    msgs = [b"abc", b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
            b"a" * 1_000_000, b""]
    msgs += [bytes(rng.integers(0, 256, n, dtype=np.uint8)) for n in
             list(range(50, 75)) + list(range(115, 135)) + [1000, 4095, 4096, 4097, 65537]]
    paths = []
    for i, m in enumerate(msgs):
        p = tmp_path / f"m{i}.bin"
        p.write_bytes(m)
        paths.append(str(p))
    got = run(driver, "sha256", *paths).split()
    want = [hashlib.sha256(m).hexdigest() for m in msgs]
    assert got == want
    # The FIPS 180-4 published digests themselves.
    assert got[0] == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert got[1] == "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    assert got[2] == "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"
