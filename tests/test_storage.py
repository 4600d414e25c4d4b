"""K3X storage records on the CPU: the oracle's CRC32C and FNV-1a 64 against
their published check values and the reference's CRC32C compiled in place
(runtime/src/crc32c.cpp; tests/cpp/test_checksums.cpp:11-16 holds the
standard vector), and the reader's open-time checks (runtime/src/reader.cpp
:414-560) on fixtures written from K3X_FORMAT.md.  Opening is host work; the
device side is tests/test_gpu_storage.py."""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from golden.k3x_fixture import fnv1a64, write_k3x


def test_crc32c_known_answers(oracle):
    assert oracle.crc32c(b"123456789") == 0xE3069283  # test_checksums.cpp:13, RFC 3720
    assert oracle.crc32c(b"") == 0
    assert oracle.crc32c(bytes(32)) == 0x8A9136AA     # RFC 3720 B.4: 32 zero bytes
    assert oracle.crc32c(b"\xff" * 32) == 0x62A8AB43  # RFC 3720 B.4: 32 0xFF bytes
    assert oracle.crc32c(bytes(range(32))) == 0x46DD794E


def test_crc32c_vs_reference(oracle, reflib):
    rng = np.random.default_rng(3)
    for n in (1, 7, 4095, 4096, 4097, 100_003):
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert oracle.crc32c(data) == reflib.crc32c(data)


def test_crc32c_table_method(oracle):
    """The byte-table restatement the bench times (k3xo_crc32c_table, the
    method of runtime/src/crc32c.cpp) gives the bit-at-a-time value, the
    RFC 3720 check values included."""
    assert oracle.crc32c_table(b"123456789") == 0xE3069283
    assert oracle.crc32c_table(b"") == 0
    assert oracle.crc32c_table(bytes(32)) == 0x8A9136AA
    rng = np.random.default_rng(4)
    for n in (1, 2, 255, 4096, 65_537):
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert oracle.crc32c_table(data) == oracle.crc32c(data)


def test_fnv1a64_known_answers(oracle):
    # Published FNV-1a 64 values (Fowler/Noll/Vo test suite).
    assert oracle.fnv1a64("") == 0xCBF29CE484222325
    assert oracle.fnv1a64("a") == 0xAF63DC4C8601EC8C
    assert oracle.fnv1a64("foobar") == 0x85944171F73967E8
    name = "model.layers.1.feed_forward.experts.0.gate"
    assert fnv1a64(name) == oracle.fnv1a64(name)


def small_tensors(oracle, inter=128, hidden=256):
    rng = np.random.default_rng(5)
    ex = {f"{r}_packed": rng.integers(0, 256, inter * hidden // 2, dtype=np.uint8)
          for r in ("gate", "up", "down")}
    ex.update({f"{r}_scales": rng.integers(119, 124, inter * hidden // 32, dtype=np.uint8)
               for r in ("gate", "up", "down")})
    from golden.k3x_fixture import expert_tensors
    return expert_tensors(1, 0, ex, inter, hidden)


def open_status(path):
    import k3x_amd
    s = k3x_amd.Storage(path)
    st = s.open_status
    s.close()
    return st


def rewrite(path, at, data, fix_crc, oracle):
    b = bytearray(open(path, "rb").read())
    b[at:at + len(data)] = data
    if fix_crc:
        struct.pack_into("<I", b, 4092, oracle.crc32c(bytes(b[:4092])))
    open(path, "wb").write(bytes(b))


def reader_cases(oracle, tmp_path):
    """K3X files and the status reader.cpp gives each: a good file, the
    superblock field cases, a truncated file, overlapping and unaligned
    extents, a duplicate tensor id and a missing file."""
    crc = oracle.crc32c
    out = []
    good = str(tmp_path / "good.k3x")
    write_k3x(good, small_tensors(oracle), crc)
    out.append((good, 0))
    cases = {  # (offset, bytes, recompute the superblock CRC) -> reader.cpp status
        "magic": (0, b"K3XCHKPX", True, 2),
        "version": (8, struct.pack("<H", 2), True, 3),
        "superblock_crc": (1000, b"\x01", False, 6),
        "required_feature": (24, struct.pack("<Q", 1), True, 4),
        "reserved": (1000, b"\x01", True, 8),
        "not_finalized": (20, struct.pack("<I", 0), True, 7),
    }
    for name, (at, data, fix, want) in cases.items():
        p = str(tmp_path / f"{name}.k3x")
        write_k3x(p, small_tensors(oracle), crc)
        rewrite(p, at, data, fix, oracle)
        out.append((p, want))
    # Truncated: the declared length no longer matches.
    p = str(tmp_path / "short.k3x")
    write_k3x(p, small_tensors(oracle), crc)
    b = open(p, "rb").read()
    open(p, "wb").write(b[:-4096])
    out.append((p, 7))
    # Overlapping and unaligned extents; a duplicate tensor id.
    t = small_tensors(oracle)
    layout = write_k3x(str(tmp_path / "probe.k3x"), t, crc)
    tens = layout["dirs"][0]
    p = str(tmp_path / "overlap.k3x")
    write_k3x(p, t, crc)
    rewrite(p, tens + 16 + 128 + 64, struct.pack("<Q", layout["payload"][0]), False, oracle)
    out.append((p, 9))
    p = str(tmp_path / "unaligned.k3x")
    write_k3x(p, t, crc)
    rewrite(p, tens + 16 + 64, struct.pack("<Q", layout["payload"][0] + 16), False, oracle)
    out.append((p, 9))
    p = str(tmp_path / "dup.k3x")
    t2 = small_tensors(oracle)
    t2[1]["id"] = fnv1a64(t2[0]["name"])
    write_k3x(p, t2, crc)
    out.append((p, 8))
    out.append((str(tmp_path / "absent.k3x"), 1))
    return out


def test_reader_open_checks(oracle, tmp_path):
    import k3x_amd
    for path, want in reader_cases(oracle, tmp_path):
        assert open_status(path) == want, os.path.basename(path)
    del k3x_amd


def test_reader_checksum_verification(oracle, tmp_path):
    """k3x_hip_storage_verify: Reader::open's checksums mode
    (runtime/src/reader.cpp:672-721) in its order -- tensor data and
    auxiliary CRC32C, the directories' SHA-256, the whole file's SHA-256 --
    on a good file (digests written with Python's hashlib, an independent
    SHA-256) and on one file per failing check."""
    import k3x_amd
    crc = oracle.crc32c
    t = small_tensors(oracle)
    good = str(tmp_path / "good.k3x")
    layout = write_k3x(good, t, crc)
    cases = [(good, 0)]
    p = str(tmp_path / "dir_digest.k3x")
    write_k3x(p, t, crc, bad_directory_digest=True)
    cases.append((p, 12))
    p = str(tmp_path / "root_digest.k3x")
    write_k3x(p, t, crc, bad_root_digest=True)
    cases.append((p, 13))
    # A payload byte changed: the data CRC fails first (the digests too).
    p = str(tmp_path / "data.k3x")
    write_k3x(p, t, crc)
    rewrite(p, layout["payload"][0] + 5, b"\x5a", False, oracle)
    cases.append((p, 10))
    # A scale byte of the second extent: the auxiliary CRC.
    p = str(tmp_path / "aux.k3x")
    write_k3x(p, t, crc)
    b = bytearray(open(p, "rb").read())
    at = layout["payload"][1] + 3
    b[at] ^= 0x01
    open(p, "wb").write(bytes(b))
    cases.append((p, 11))
    for path, want in cases:
        s = k3x_amd.Storage(path)
        assert s.open_status == 0, os.path.basename(path)
        assert s.verify() == want, os.path.basename(path)
        s.close()
