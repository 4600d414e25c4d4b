"""K3X storage records on the GPU: k3x_hip_crc32c against the oracle's
CRC32C (itself pinned to the published check values and to the reference's
crc32c.cpp, tests/test_storage.py) over ragged and multi-chunk sizes, and
k3x_hip_storage_upload_expert (load_storage_expert, runtime/src/
storage_slice.cpp:42-92) against a host upload of the same expert: the bank
slots dequantise bit-identically, the load's ordered SHA-256 equals
hashlib's over the six extents, and a layer call through each gives the
same output; corrupted CRCs, a missing tensor, a wrong shape and a file
without the STORAGE_FIXTURE feature are rejected with the reader's codes."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from golden.k3x_fixture import expert_tensors, write_k3x

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def say(msg):
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def hip():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import k3x_amd
    ctx = k3x_amd.Context(0)
    yield k3x_amd, ctx
    ctx.close()


@pytest.mark.parametrize("n", [0, 1, 15, 16, 4095, 4096, 4097, 65536 + 48, 5_505_024,
                               23_396_352 + 16])
def test_device_crc32c(hip, oracle, n):
    k3x_amd, ctx = hip
    say(f"crc32c n={n}")
    rng = np.random.default_rng(n)
    host = rng.integers(0, 256, max(n, 16), dtype=np.uint8)
    dev = torch.from_numpy(host).to("cuda:0")
    st, crc = ctx.crc32c(dev, n)
    assert st == 0 and crc == oracle.crc32c(host[:n].tobytes())


@pytest.mark.parametrize("n", [16, 4096 + 16, 8192 * 512 * 16 + 48, (64 << 20) + 32])
def test_stream_read_fold(hip, n):
    """k3x_hip_stream_read (the bench's read-ceiling measurement) reads every
    word exactly once: its XOR fold equals numpy's over the same words, for
    sizes below, at and past one word per thread of the full grid; misaligned
    or ragged extents are rejected."""
    k3x_amd, ctx = hip
    say(f"stream_read n={n}")
    rng = np.random.default_rng(n)
    host = rng.integers(0, 1 << 32, n // 4, dtype=np.uint32)
    dev = torch.from_numpy(host.view(np.int32)).to("cuda:0")
    fold = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    assert ctx.stream_read(dev, fold, n) == 0
    assert ctx.synchronize() == 0
    assert int(fold.cpu().numpy().view(np.uint32)[0]) == int(np.bitwise_xor.reduce(host))
    assert ctx.stream_read(dev, fold, n - 4) == k3x_amd.ERR_INVALID_EXTENT
    assert ctx.stream_read(dev[1:], fold, 16) == k3x_amd.ERR_INVALID_EXTENT


def make_expert(seed, inter, hidden):
    rng = np.random.default_rng(seed)
    ex = {f"{r}_packed": rng.integers(0, 256, inter * hidden // 2, dtype=np.uint8)
          for r in ("gate", "up", "down")}
    ex.update({f"{r}_scales": rng.integers(119, 124, inter * hidden // 32, dtype=np.uint8)
               for r in ("gate", "up", "down")})
    return ex


@pytest.mark.parametrize("hidden,inter", [(256, 128), (7168, 2048)])
def test_storage_upload(hip, oracle, tmp_path, hidden, inter):
    k3x_amd, ctx = hip
    say(f"storage upload H={hidden} I={inter}")
    crc = oracle.crc32c
    experts = [make_expert(10 + e, inter, hidden) for e in range(2)]
    tensors = []
    for e, ex in enumerate(experts):
        tensors += expert_tensors(3, e, ex, inter, hidden)
    path = str(tmp_path / "experts.k3x")
    write_k3x(path, tensors, crc)
    shape = k3x_amd.LayerShape(hidden, inter, 4, 0)
    a, b = k3x_amd.Bank(ctx, shape), k3x_amd.Bank(ctx, shape)
    store = k3x_amd.Storage(path)
    assert store.open_status == 0
    import hashlib
    for e, ex in enumerate(experts):
        st, n, digest = store.upload_expert_digest(a, e, 3, e)
        assert st == 0 and n == 3 * (inter * hidden // 2 + inter * hidden // 32)
        # The ordered SHA-256 load_storage_expert returns (storage_slice.cpp:
        # 80-90): the six extents in order, against Python's hashlib.
        want = hashlib.sha256(b"".join(bytes(ex[f"{r}_{k}"]) for r in ("gate", "up", "down")
                                       for k in ("packed", "scales"))).digest()
        assert digest == want, e
        assert b.upload_expert(e, ex, tensor_ids=(100 + 3 * e, 101 + 3 * e, 102 + 3 * e)) == 0
        for m, rows in ((0, inter), (1, inter), (2, hidden)):
            ra = a.dequant_rows(e, m, 0, rows)
            rb = b.dequant_rows(e, m, 0, rows)
            assert torch.equal(ra.view(torch.int32), rb.view(torch.int32))
    # The slot's tensor ids are the records' (FNV-1a of the names).
    from golden.k3x_fixture import fnv1a64
    assert a.find(fnv1a64("model.layers.3.feed_forward.experts.1.down"))[1:] == (1, 2)
    # Rejections: missing expert, wrong layer shape, bad CRCs, no fixture bit.
    assert store.upload_expert(a, 2, 3, 7)[0] == k3x_amd.ERR_TENSOR_NOT_FOUND
    other = k3x_amd.Bank(ctx, k3x_amd.LayerShape(hidden, inter * 2, 2, 0))
    assert store.upload_expert(other, 0, 3, 0)[0] == k3x_amd.ERR_INVALID_MXFP4
    other.close()
    store.close()
    for field, want in (("data_crc", 10), ("aux_crc", 11)):
        bad = [dict(t) for t in tensors]
        bad[4][field] = (crc(bad[4]["data"] if field == "data_crc" else bad[4]["aux"]) ^ 1)
        p = str(tmp_path / f"{field}.k3x")
        write_k3x(p, bad, crc)
        s = k3x_amd.Storage(p)
        assert s.open_status == 0
        # Into the slot that holds these ids: rejected before it is touched.
        assert s.upload_expert(a, 1, 3, 1)[0] == want, field
        s.close()
        ra, rb = a.dequant_rows(1, 1, 0, inter), b.dequant_rows(1, 1, 0, inter)
        assert torch.equal(ra.view(torch.int32), rb.view(torch.int32))
    p = str(tmp_path / "plain.k3x")
    write_k3x(p, tensors, crc, optional_features=0)
    s = k3x_amd.Storage(p)
    assert s.upload_expert(a, 3, 3, 0)[0] == k3x_amd.ERR_INVALID_EXTENT
    s.close()
    a.close()
    b.close()
