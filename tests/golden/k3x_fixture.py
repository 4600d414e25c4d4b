"""Writes small K3X checkpoints for the storage tests (test infrastructure).

Layout follows K3X_FORMAT.md: 4 KiB superblock (magic K3XCHKPT, version
1.0, finalized, CRC32C over bytes 0..4091 at 4092), 4 KiB-aligned payload
extents, then the tensor (TENS, 128-byte records), layer (LAYR, 64-byte),
expert (EXPT, 64-byte) directories and the 256-byte model config, each 4 KiB
aligned.  The digests at 168..231 are those Reader::open checks with
VerifyMode::checksums (runtime/src/reader.cpp:672-721), computed here with
Python's hashlib: the SHA-256 of the four directories concatenated, and of
the whole file with bytes 200..231 and 4092..4095 taken as zeros.  `crc` is
a CRC32C function (the oracle's)."""
from __future__ import annotations

import hashlib
import struct


def _align(n: int) -> int:
    return (n + 4095) & ~4095


def fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for c in name.encode():
        h ^= c
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def expert_tensors(layer: int, expert: int, ex: dict, inter: int, hidden: int) -> list[dict]:
    """The three native MXFP4 tensors of one expert (gate/up [inter][hidden],
    down [hidden][inter]) named as runtime/src/storage_slice.cpp:50-52 names
    them."""
    base = f"model.layers.{layer}.feed_forward.experts.{expert}."
    dims = {"gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}
    return [dict(name=base + r, dtype=2, quant=1, rank=2, dims=dims[r], layer=layer,
                 expert=expert, data=bytes(ex[f"{r}_packed"]), aux=bytes(ex[f"{r}_scales"]))
            for r in ("gate", "up", "down")]


def write_k3x(path: str, tensors: list[dict], crc, optional_features: int = 1,
              layers: int = 1, required_features: int = 0, bad_directory_digest: bool = False,
              bad_root_digest: bool = False) -> dict:
    """Writes the file; returns the offsets it used (for corruption tests).
    bad_*_digest: store that digest with its first byte flipped."""
    at = 4096
    payload = []
    recs = []
    for t in tensors:
        d_off = at
        payload.append((d_off, t["data"]))
        at = _align(at + len(t["data"]))
        a_off, a_len = 0, 0
        if t.get("aux") is not None:
            a_off, a_len = at, len(t["aux"])
            payload.append((a_off, t["aux"]))
            at = _align(at + a_len)
        dims = list(t["dims"]) + [0] * (4 - len(t["dims"]))
        r = struct.pack("<QIHHBBHiiI4QQQQQQII16x", t.get("id", fnv1a64(t["name"])), 0,
                        t["dtype"], t["quant"], t["rank"], 0, 0, t["layer"], t["expert"], 0,
                        *dims, d_off, len(t["data"]), len(t["data"]) * 2, a_off, a_len,
                        t.get("data_crc", crc(t["data"])),
                        t.get("aux_crc", crc(t["aux"]) if a_len else 0))
        assert len(r) == 128
        recs.append(r)
    tens = b"TENS" + struct.pack("<IQ", 128, len(recs)) + b"".join(recs)
    layr = b"LAYR" + struct.pack("<IQ", 64, layers) + bytes(64 * layers)
    expt = b"EXPT" + struct.pack("<IQ", 64, 0)
    cfg = bytearray(256)
    struct.pack_into("<I", cfg, 8, layers)
    dirs = []
    for blob in (tens, layr, expt, bytes(cfg)):
        dirs.append((at, blob))
        at = _align(at + len(blob))
    total = at
    sb = bytearray(4096)
    sb[0:8] = b"K3XCHKPT"
    struct.pack_into("<HHIII", sb, 8, 1, 0, 4096, 4096, 1)
    struct.pack_into("<QQ", sb, 24, required_features, optional_features)
    vals = []
    for off, blob in dirs:
        vals += [off, len(blob)]
    struct.pack_into("<10Q", sb, 88, *vals, 4096, total)
    dir_digest = bytearray(hashlib.sha256(b"".join(blob for _, blob in dirs)).digest())
    if bad_directory_digest:
        dir_digest[0] ^= 0xFF
    sb[168:200] = dir_digest
    buf = bytearray(total)
    buf[:4096] = sb
    for off, blob in payload + dirs:
        buf[off:off + len(blob)] = blob
    root_digest = bytearray(hashlib.sha256(bytes(buf)).digest())  # 200..231, 4092.. still zero
    if bad_root_digest:
        root_digest[0] ^= 0xFF
    buf[200:232] = root_digest
    struct.pack_into("<I", buf, 4092, crc(bytes(buf[:4092])))
    with open(path, "wb") as f:
        f.write(buf)
    return {"payload": [o for o, _ in payload], "dirs": [o for o, _ in dirs], "total": total}
