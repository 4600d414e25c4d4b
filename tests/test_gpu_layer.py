"""GPU parity of the HIP MoE layer against the CPU oracle (through the C ABI).

Standards of the layer contract:
* bit-exact: dequantised weights (fp32 bits, including -0.0 and overflow),
  RMSNorm output, router logits, Top-K ids and weights, expert-major CSR and
  first-use order;
* fp32 outputs before the bf16 cast within rtol 2e-3 / atol 1e-3, and each
  bf16 output within 1 bf16 ulp of the bf16 cast of the oracle's fp32 output
  or, where the value is so close to zero that a bf16 ulp is finer than the
  absolute tolerance, within atol 1e-3 of it (comparing two bf16 casts of
  nearly equal fp32 values, a rounding-boundary flip is one ulp);
* stage isolation: the down projection and combine are checked on the GPU's
  own activations so accumulation-order differences are not compounded.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle import bf16_bits, bf16_to_f32

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

RTOL, ATOL = 2e-3, 1e-3


def say(msg: str) -> None:
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


def ulp_diff_bf16(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """|a - b| in bf16 ulps for same-sign finite values (sign change counts big)."""
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    a = np.where(a & 0x8000, 0x8000 - a, a)
    b = np.where(b & 0x8000, 0x8000 - b, b)
    return np.abs(a - b)


def to_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


# ---------------------------------------------------------------------------
# Exhaustive dequantisation: all 16 codes under every legal E8M0 scale.
# ---------------------------------------------------------------------------
def test_dequant_exhaustive_bitexact(hip, oracle):
    k3x_amd, ctx = hip
    H, I = 512, 128  # gate/up [128 x 512] -> 2048 scale blocks
    say("dequant exhaustive: bank H=512 I=128 E=1")
    shape = k3x_amd.LayerShape(hidden=H, inter=I, experts=1)
    bank = k3x_amd.Bank(ctx, shape)
    rng = np.random.default_rng(7)
    n = H * I
    blocks = n // 32
    # gate: every block holds codes 0..15 twice, block b has scale b % 255.
    gate_packed = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8),
                          n // 16)
    gate_scales = (np.arange(blocks) % 255).astype(np.uint8)
    ex = dict(gate_packed=gate_packed, gate_scales=gate_scales,
              up_packed=rng.integers(0, 256, n // 2, dtype=np.uint8),
              up_scales=rng.integers(0, 255, blocks, dtype=np.uint8),
              down_packed=rng.integers(0, 256, n // 2, dtype=np.uint8),
              down_scales=rng.integers(0, 255, blocks, dtype=np.uint8))
    assert bank.upload_expert(0, ex) == 0
    for m, (pk, sc, rows, cols) in enumerate([
            (ex["gate_packed"], ex["gate_scales"], I, H),
            (ex["up_packed"], ex["up_scales"], I, H),
            (ex["down_packed"], ex["down_scales"], H, I)]):
        st, want = oracle.decode_mxfp4(pk, sc, rows, cols, 32)
        assert st == 0
        got = to_np(bank.dequant_rows(0, m, 0, rows))
        mism = np.count_nonzero(got.view(np.uint32) != want.view(np.uint32))
        say(f"matrix {m}: {mism} bit mismatches of {got.size}")
        assert mism == 0
    bank.close()


def test_upload_rejects_reserved_scale(hip):
    k3x_amd, ctx = hip
    shape = k3x_amd.LayerShape(hidden=128, inter=128, experts=1)
    bank = k3x_amd.Bank(ctx, shape)
    n = 128 * 128
    ex = dict(gate_packed=np.zeros(n // 2, np.uint8), gate_scales=np.full(n // 32, 127, np.uint8),
              up_packed=np.zeros(n // 2, np.uint8), up_scales=np.full(n // 32, 127, np.uint8),
              down_packed=np.zeros(n // 2, np.uint8), down_scales=np.full(n // 32, 127, np.uint8))
    ex["down_scales"][5] = 0xFF
    assert bank.upload_expert(0, ex) == k3x_amd.ERR_INVALID_MXFP4
    ex["down_scales"][5] = 127
    assert bank.upload_expert(0, ex, tensor_ids=(0, 1, 2)) == k3x_amd.ERR_INVALID_MXFP4
    assert bank.upload_expert(0, ex, tensor_ids=(5, 5, 6)) == k3x_amd.ERR_INVALID_MXFP4
    assert bank.upload_expert(0, ex, tensor_ids=(5, 6, 7)) == 0
    assert bank.find(6) == (0, 0, 1)
    assert bank.find(99)[0] == k3x_amd.ERR_TENSOR_NOT_FOUND
    bank.close()


# ---------------------------------------------------------------------------
# Full layer on the seeded benchmark configurations.
# ---------------------------------------------------------------------------
def run_layer(k3x_amd, ctx, cfg, bank, x_bits):
    dev = "cuda:0"
    T, H, I, E, K = cfg.tokens, cfg.hidden, cfg.inter, cfg.experts, cfg.top_k
    x = torch.from_numpy(x_bits.view(np.int16)).to(dev)
    out = torch.empty((T, H), dtype=torch.int16, device=dev)
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device=dev)
    taps = dict(normed_x=z((T, H), torch.int16), logits=z((T, E), torch.float32),
                ids=z((T, K), torch.int32), weights=z((T, K), torch.float32),
                counts=z((E,), torch.int32), offsets=z((E + 1,), torch.int32),
                pair_token=z((T * K,), torch.int32), pair_slot=z((T * K,), torch.int32),
                first_use=z((E,), torch.int32), n_active=z((1,), torch.int32),
                active_first_use=z((E,), torch.int32), act=z((T * K, I), torch.int16),
                expert_out=z((T, K, H), torch.float32), out_f32=z((T, H), torch.float32))
    if cfg.shared_inter:
        taps["shared_out"] = z((T, H), torch.float32)
    params = k3x_amd.make_params(T, K, cfg.routed_scale, cfg.eps, cfg.glu, cfg.beta, cfg.linear,
                                 cfg.renorm)
    st = k3x_amd.moe_forward(ctx, bank, params, x, out, taps)
    assert st == 0, st
    assert ctx.synchronize() == 0
    got = {k: to_np(v) for k, v in taps.items()}
    got["out"] = to_np(out)
    for k in ("ids", "counts", "offsets", "pair_token", "pair_slot", "first_use", "n_active",
              "active_first_use"):
        got[k] = got[k].view(np.uint32)
    for k in ("normed_x", "act", "out"):
        got[k] = got[k].view(np.uint16)
    return got


def check_layer(oracle, layer, got, tokens_checked=None):
    cfg = layer.cfg
    T, K, E = cfg.tokens, cfg.top_k, cfg.experts
    x_bits = layer.x_bits()
    # RMSNorm, bit-exact.
    xn = layer.normed(x_bits)
    xn_bits = (xn.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(got["normed_x"], xn_bits), "RMSNorm output differs"
    say("rmsnorm bit-exact")
    # Router logits, ids, weights: bit-exact.
    logits, ids, w = layer.route(xn)
    assert np.array_equal(got["logits"].view(np.uint32), logits.view(np.uint32)), "logits differ"
    assert np.array_equal(got["ids"], ids), "Top-K ids differ"
    assert np.array_equal(got["weights"].view(np.uint32), w.view(np.uint32)), "weights differ"
    say("router logits / ids / weights bit-exact")
    # Grouping: CSR + first-use order, bit-exact; same groups as the plan.
    st, csr = oracle.expert_major_csr(ids, E)
    assert st == 0
    for k in ("counts", "offsets", "first_use"):
        assert np.array_equal(got[k], csr[k]), k
    P = T * K
    assert np.array_equal(got["pair_token"][:P], csr["pair_token"])
    assert np.array_equal(got["pair_slot"][:P], csr["pair_slot"])
    na = int(got["n_active"][0])
    assert na == csr["n_active"]
    assert np.array_equal(got["active_first_use"][:na], csr["active_first_use"])
    st, plan = oracle.expert_major_plan(ids, w)
    assert st == 0
    assert np.array_equal(plan["group_expert"], csr["active_first_use"])
    say(f"grouping bit-exact ({na} active experts)")
    # Per-pair activations and outputs.
    tokens = range(T) if tokens_checked is None else tokens_checked
    act_ref, y_ref = layer.pair_outputs(xn, ids, tokens)
    act_gpu = got["act"]  # CSR rows
    worst_act = 0
    for r in range(P):
        t, s = int(csr["pair_token"][r]), int(csr["pair_slot"][r])
        if t not in tokens:
            continue
        ref_bits = (act_ref[t, s].view(np.uint32) >> 16).astype(np.uint16)
        d = ulp_diff_bf16(act_gpu[r], ref_bits)
        worst_act = max(worst_act, int(d.max()))
        frac = np.count_nonzero(d) / d.size
        assert frac < 0.02, f"pair ({t},{s}): {frac:.4f} of activations off"
    assert worst_act <= 1, f"activation off by {worst_act} bf16 ulps"
    say(f"activations within {worst_act} bf16 ulp")
    # Down projection on the GPU's own activations (isolates the GEMM).
    for r in range(P):
        t, s = int(csr["pair_token"][r]), int(csr["pair_slot"][r])
        if t not in tokens:
            continue
        e = int(ids[t, s])
        ex = layer.expert(e)
        a = bf16_to_f32(act_gpu[r])
        st, yd = oracle.mxfp4_matvec(a, ex["down_packed"], ex["down_scales"], cfg.hidden,
                                     cfg.inter, 32)
        np.testing.assert_allclose(got["expert_out"][t, s], yd, rtol=1e-4, atol=1e-4)
    say("down projection matches on GPU activations")
    # Against the fully independent CPU layer.
    shared = layer.shared_out(xn, tokens)
    if cfg.shared_inter:
        for t in tokens:
            np.testing.assert_allclose(got["shared_out"][t], shared[t], rtol=RTOL, atol=ATOL)
    out_ref = layer.combine(y_ref, w, shared, tokens)
    for t in tokens:
        np.testing.assert_allclose(got["out_f32"][t], out_ref[t], rtol=RTOL, atol=ATOL)
        ref_bits = bf16_bits(out_ref[t])
        d = ulp_diff_bf16(got["out"][t], ref_bits)
        near = np.abs(bf16_to_f32(got["out"][t]) - bf16_to_f32(ref_bits)) <= ATOL
        bad = (d > 1) & ~near
        assert not bad.any(), f"token {t}: {int(bad.sum())} bf16 outputs off by > 1 ulp"
        say(f"token {t}: bf16 max ulp {int(d.max())} (all > 1 ulp within atol)")
    # Combine on the GPU's own per-pair outputs: bit-exact.
    comb = layer.combine(got["expert_out"], w,
                         got["shared_out"] if cfg.shared_inter else np.zeros_like(got["out_f32"]))
    assert np.array_equal(comb.view(np.uint32), got["out_f32"].view(np.uint32))
    say("layer output within tolerance; ordered combine bit-exact")


def make_bank(k3x_amd, ctx, cfg):
    shape = k3x_amd.LayerShape(cfg.hidden, cfg.inter, cfg.experts, cfg.shared_inter)
    bank = k3x_amd.Bank(ctx, shape)
    bank.fill_synthetic(cfg.seed, cfg.scale_lo, cfg.scale_hi, cfg.router_sigma, cfg.bias_sigma,
                        cfg.shared_sigma, 1.0)
    return bank


@pytest.mark.parametrize("cid", [1, 3])
def test_layer_parity(hip, oracle, cid):
    from synth import CONFIGS, SynthLayer
    k3x_amd, ctx = hip
    cfg = CONFIGS[cid]
    say(f"layer parity config {cid} ({cfg.name}) T={cfg.tokens} E={cfg.experts}")
    bank = make_bank(k3x_amd, ctx, cfg)
    layer = SynthLayer(oracle, cfg)
    # Synthetic fill is bit-identical to the CPU generator (sampled rows).
    for e in (0, cfg.experts - 1):
        ex = layer.expert(e)
        st, want = oracle.decode_mxfp4(ex["down_packed"][: 4 * cfg.inter // 2],
                                       ex["down_scales"][: 4 * cfg.inter // 32], 4, cfg.inter)
        got = to_np(bank.dequant_rows(e, 2, 0, 4))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got = run_layer(k3x_amd, ctx, cfg, bank, layer.x_bits())
    check_layer(oracle, layer, got)
    bank.close()
