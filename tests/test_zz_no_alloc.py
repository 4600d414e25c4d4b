"""k3x_hip_moe_forward_noalloc against k3x_hip_moe_forward through the C ABI.

The no-allocation entry point runs the same kernels over a fixed device
array instead of the context's grow-only scratch, so its results must be
bit-identical: two calls in a row, the second with fewer tokens, on the
decode path (T <= 4) and on the general path, then a call whose buffers do
not fit the array, which is refused before anything is enqueued.  Each
no-allocation call runs first on its context (before any allocating call
could have grown the context's scratch) and must leave the context's
scratch (0 on the first call) and the bank's bytes unchanged.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TAPS = ("normed_x", "logits", "ids", "weights", "counts", "offsets", "pair_token",
        "pair_slot", "first_use", "n_active", "active_first_use", "act", "expert_out",
        "shared_out", "out_f32", "shared_act")


def say(msg: str) -> None:
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


def call(k3x_amd, ctx, bank, cfg, x_bits, flags, noalloc):
    dev = "cuda:0"
    scratch0, bank_bytes0 = ctx.stats().scratch_bytes, bank.bytes()
    T, H, I, E, K, S = cfg
    x = torch.from_numpy(np.ascontiguousarray(x_bits).view(np.int16)).to(dev)
    out = torch.full((T, H), -1, dtype=torch.int16, device=dev)
    z = lambda shape, dt: torch.full(shape, -1, dtype=dt, device=dev)
    taps = dict(normed_x=z((T, H), torch.int16), logits=z((T, E), torch.float32),
                ids=z((T, K), torch.int32), weights=z((T, K), torch.float32),
                counts=z((E,), torch.int32), offsets=z((E + 1,), torch.int32),
                pair_token=z((T * K,), torch.int32), pair_slot=z((T * K,), torch.int32),
                first_use=z((E,), torch.int32), n_active=z((1,), torch.int32),
                active_first_use=z((E,), torch.int32), act=z((T * K, I), torch.int16),
                expert_out=z((T, K, H), torch.float32), shared_out=z((T, H), torch.float32),
                out_f32=z((T, H), torch.float32), shared_act=z((T, S), torch.int16))
    params = k3x_amd.make_params(T, K, 2.5, 1e-6, k3x_amd.GLU_SWIGLU, 4.0, None,
                                 k3x_amd.RENORM_FLOAT, flags)
    fwd = k3x_amd.moe_forward_noalloc if noalloc else k3x_amd.moe_forward
    assert fwd(ctx, bank, params, x, out, taps) == 0
    assert ctx.synchronize() == 0
    torch.cuda.synchronize()
    if noalloc:
        # Nothing allocated by the call: the context's grow-only scratch and
        # the bank's device bytes are unchanged.
        assert ctx.stats().scratch_bytes == scratch0, "context scratch grew"
        assert bank.bytes() == bank_bytes0, "bank grew"
    got = {k: v.cpu().numpy() for k, v in taps.items()}
    got["out"] = out.cpu().numpy()
    return got


@pytest.mark.parametrize("general", [False, True], ids=["decode_path", "general_path"])
def test_noalloc_matches_forward(general, oracle):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import k3x_amd
    ctx = k3x_amd.Context(0)
    H, I, E, K, S = 1024, 512, 64, 8, 256
    bank = k3x_amd.Bank(ctx, k3x_amd.LayerShape(H, I, E, S))
    bank.fill_synthetic(0x5107, 119, 123, 0.02, 0.1, 0.02, 1.0)
    flags = k3x_amd.FLAG_GENERAL_PATH if general else 0
    assert ctx.stats().scratch_bytes == 0  # a fresh context: no scratch yet
    for i, T in enumerate((4, 2) if not general else (40, 9)):
        x = oracle.synth_normal_bf16(oracle.stream_key(0xA110C + i, 12 << 32), T * H,
                                     1.0).reshape(T, H)
        cfg = (T, H, I, E, K, S)
        a = call(k3x_amd, ctx, bank, cfg, x, flags, noalloc=True)
        b = call(k3x_amd, ctx, bank, cfg, x, flags, noalloc=False)
        P = T * K
        for k in TAPS + ("out",):
            ga, gb = a[k], b[k]
            if k in ("pair_token", "pair_slot", "act"):
                ga, gb = ga[:P], gb[:P]
            if k == "active_first_use":
                n = int(a["n_active"][0])
                ga, gb = ga[:n], gb[:n]
            assert np.array_equal(ga.view(np.uint8), gb.view(np.uint8)), f"call {i} T={T}: {k}"
        say(f"call {i} T={T} general={general}: no-alloc output bit-identical")
    # Buffers beyond the fixed array: refused, nothing enqueued.
    T = 4096
    x = torch.zeros((T, H), dtype=torch.int16, device="cuda:0")
    out = torch.empty((T, H), dtype=torch.int16, device="cuda:0")
    params = k3x_amd.make_params(T, K, 2.5, 1e-6, k3x_amd.GLU_SWIGLU, 4.0, None,
                                 k3x_amd.RENORM_FLOAT, flags)
    assert k3x_amd.moe_forward_noalloc(ctx, bank, params, x, out) == k3x_amd.ERR_INVALID_EXTENT
    assert ctx.synchronize() == 0
    bank.close()
    ctx.close()
