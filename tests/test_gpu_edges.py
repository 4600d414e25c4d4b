"""GPU edge cases of the layer contract, through the C ABI.

* Top-K ties go to the lower expert index (runtime/src/official_moe.cpp:226-232,
  runtime/src/routing_policy.cpp:83-87), on every device Top-K: the decode
  path's select kernel (up to 512 experts), the general path's threshold
  Top-K for few tokens (257 to 512 and 513 to 1024 experts), its register
  Top-K with 4, 8 and 16 keys per lane (up to 256, 512 and 1024 experts; more
  than 256 tokens past 256 experts) and the LDS Top-K past 1024 experts.  Two kinds of tie: every score equal (zero
  input, equal bias: ids 0..K-1, weights routed_scale / K), and planted groups
  of duplicated router rows with equal bias, within one lane and across
  lanes, straddling the K boundary (the lower ids are selected, in order).
* The official route's all-zero-logit known answer of
  tests/cpp/test_official_moe.cpp:101-109 (ids {0, 1}, contributions .5/.5).
* Non-finite input and router scores are rejected through the latched status:
  x with a NaN or an infinity is K3X_ERR_INVALID_MXFP4 (the reference's
  finiteness check of resident_mxfp4_moe_layer, runtime/cuda/backend_cuda.cu:
  1884-1942), a non-finite bias is K3X_ERR_INVALID_STATE (routing_policy.cpp:
  40-58); the error is returned once by k3x_hip_ctx_synchronize and the next
  call on the context succeeds.
"""
from __future__ import annotations

import dataclasses
import sys

import numpy as np
import pytest

from oracle import GLU_SWIGLU, RENORM_DOUBLE, RENORM_FLOAT, SIGMOID_CR, bf16_bits

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


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


def to_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def small_layer(k3x_amd, ctx, oracle, T, E, K, shared=0, seed=0x77):
    from synth import Config, SynthLayer
    cfg = Config(f"edge_{T}_{E}_{K}", T, 256, 128, E, K, shared, 119, 123, routed_scale=2.5,
                 seed=seed)
    layer = SynthLayer(oracle, cfg)
    bank = k3x_amd.Bank(ctx, k3x_amd.LayerShape(cfg.hidden, cfg.inter, E, shared))
    bank.fill_synthetic(cfg.seed, cfg.scale_lo, cfg.scale_hi, cfg.router_sigma, cfg.bias_sigma,
                        cfg.shared_sigma, 1.0)
    return cfg, layer, bank


def route_taps(k3x_amd, ctx, cfg, bank, x_bits, flags):
    dev = "cuda:0"
    T, H, K = cfg.tokens, cfg.hidden, cfg.top_k
    x = torch.from_numpy(np.ascontiguousarray(x_bits).view(np.int16)).to(dev)
    out = torch.empty((T, H), dtype=torch.int16, device=dev)
    taps = dict(ids=torch.empty((T, K), dtype=torch.int32, device=dev),
                weights=torch.empty((T, K), dtype=torch.float32, device=dev),
                logits=torch.empty((T, cfg.experts), dtype=torch.float32, device=dev))
    params = k3x_amd.make_params(T, K, cfg.routed_scale, cfg.eps, GLU_SWIGLU, 4.0, None,
                                 cfg.renorm, flags)
    assert k3x_amd.moe_forward(ctx, bank, params, x, out, taps) == 0
    assert ctx.synchronize() == 0
    return {k: to_np(v) for k, v in taps.items()}


# (tokens, experts, general path): the Top-K kernel each case runs.
TOPK_CASES = {
    "decode_select_e384": (2, 384, False),
    "reg4_e200": (3, 200, True),
    "thr2_e384": (2, 384, True),
    "thr4_e1000": (2, 1000, True),
    "reg8_e384": (300, 384, True),
    "reg16_e1000": (300, 1000, True),
    "lds_e1100": (2, 1100, True),
}


@pytest.mark.parametrize("case", list(TOPK_CASES))
def test_topk_all_scores_tie(hip, oracle, case, parity_report):
    """Zero input -> zero logits -> every sigmoid score 0.5; equal bias: every
    adjusted score ties, so the Top-K is experts 0..K-1 in order with weights
    0.5 / (K * 0.5) * routed_scale."""
    k3x_amd, ctx = hip
    T, E, general = TOPK_CASES[case]
    K = 16
    cfg, layer, bank = small_layer(k3x_amd, ctx, oracle, T, E, K)
    layer.bias = np.full(E, 0.125, np.float32)
    assert bank.upload_router(layer.router, layer.bias, layer.gamma) == 0
    x = np.zeros((T, cfg.hidden), np.uint16)
    got = route_taps(k3x_amd, ctx, cfg, bank, x,
                     k3x_amd.FLAG_GENERAL_PATH if general else 0)
    assert not got["logits"].any()
    ids = got["ids"].view(np.uint32)
    want_w = np.float32(np.float32(0.5) / np.float32(K * 0.5)) * np.float32(2.5)
    for t in range(T):
        assert list(ids[t]) == list(range(K)), f"token {t}: {ids[t]}"
        assert (got["weights"][t] == want_w).all()
    parity_report(f"E={E}: all-tie ids 0..{K - 1}, weights {want_w!r}")
    bank.close()


@pytest.mark.parametrize("case", list(TOPK_CASES))
def test_topk_planted_ties(hip, oracle, case, parity_report):
    """Groups of experts with identical router rows and identical bias tie
    exactly (the logits of identical rows are bit-identical).  Group A (bias
    +5) has four members, two of them in the same lane (e and e + 64); group
    B (bias +4) has three; K = 6 takes all of A and the two lowest ids of B,
    in that order.  The oracle's route over the GPU's logits (the reference's
    comparator) must agree bit for bit."""
    k3x_amd, ctx = hip
    T, E, general = TOPK_CASES[case]
    K = 6
    cfg, layer, bank = small_layer(k3x_amd, ctx, oracle, T, E, K, seed=0x99 + E)
    rng = np.random.default_rng(E)
    group_a = [5, 69, min(133, E - 1), 37]     # 5 and 69 share lane 5
    group_b = sorted(rng.choice(np.arange(140, E), 3, replace=False).tolist())
    router = layer.router.copy()
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    for grp, b in ((group_a, 5.0), (group_b, 4.0)):
        for e in grp:
            router[e] = router[grp[0]]
            bias[e] = b
    layer.router, layer.bias = router, bias
    assert bank.upload_router(router, bias, layer.gamma) == 0
    x = layer.x_bits()
    got = route_taps(k3x_amd, ctx, cfg, bank, x, k3x_amd.FLAG_GENERAL_PATH if general else 0)
    ids = got["ids"].view(np.uint32)
    want = sorted(group_a) + group_b[:2]
    for t in range(T):
        lg = got["logits"][t]
        for grp in (group_a, group_b):
            assert len({lg[e].tobytes() for e in grp}) == 1, "planted rows must tie"
        assert list(ids[t]) == want, f"token {t}: {list(ids[t])} != {want}"
        st, rid, rw, _ = oracle.route(lg, bias, K, RENORM_FLOAT, 2.5, SIGMOID_CR)
        assert st == 0 and list(rid) == want
        assert np.array_equal(rw.view(np.uint32), got["weights"][t].view(np.uint32))
    parity_report(f"E={E}: planted ties -> ids {want} (lower index first)")
    bank.close()


def test_official_route_all_zero_logits(hip):
    """tests/cpp/test_official_moe.cpp:101-109: three experts, zero logits and
    zero correction, Top-2 -> ids {0, 1}, contributions {0.5, 0.5}.  Here the
    zero logits come from a zero router over the prepared hidden."""
    k3x_amd, ctx = hip
    H, L, I, E, K, T = 128, 128, 128, 3, 2, 2
    bank = k3x_amd.Bank(ctx, k3x_amd.LayerShape(L, I, E, 0))
    bank.fill_synthetic(5, 121, 125)
    off = k3x_amd.Official(ctx, bank, H, 0)
    z16 = lambda *s: np.zeros(s, np.uint16)
    one16 = lambda n: np.full(n, 0x3F80, np.uint16)  # bf16 1.0
    assert off.upload_ffn(z16(L, H), one16(L), z16(H, L)) == 0
    assert off.upload_route(one16(H), z16(H), one16(H), z16(E, H), np.zeros(E, np.float32)) == 0
    dev = "cuda:0"
    rng = np.random.default_rng(3)
    prefix = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dev)
    residual = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dev)
    hidden = torch.empty((T, H), dtype=torch.int16, device=dev)
    assert off.prepare(T, 1e-5, prefix, residual, hidden) == 0
    params = k3x_amd.make_params(T, K, 1.0, 1e-5, k3x_amd.GLU_SITU, 4.0, 25.0,
                                 k3x_amd.RENORM_DOUBLE)
    taps = dict(ids=torch.empty((T, K), dtype=torch.int32, device=dev),
                contributions=torch.empty((T, K), dtype=torch.float32, device=dev),
                logits=torch.empty((T, E), dtype=torch.float32, device=dev))
    out = torch.empty((T, H), dtype=torch.int16, device=dev)
    assert off.ffn(params, hidden, prefix, out, taps=taps) == 0
    assert ctx.synchronize() == 0
    assert not to_np(taps["logits"]).any()
    ids = to_np(taps["ids"]).view(np.uint32)
    c = to_np(taps["contributions"])
    for t in range(T):
        assert list(ids[t]) == [0, 1]
        assert list(c[t]) == [0.5, 0.5]
    off.close()
    bank.close()


@pytest.mark.parametrize("general", [False, True], ids=["decode_path", "general_path"])
@pytest.mark.parametrize("bad", ["nan", "inf", "neg_inf"])
def test_nonfinite_input_rejected(hip, oracle, general, bad):
    """A non-finite element of x: the call is accepted (it runs on the stream),
    the kernels latch K3X_ERR_INVALID_MXFP4 and skip the rest of the layer,
    k3x_hip_ctx_synchronize returns it once; the next call on the context
    succeeds and is bit-identical to the same call on a fresh state."""
    k3x_amd, ctx = hip
    T, E, K = 2, 64, 4
    cfg, layer, bank = small_layer(k3x_amd, ctx, oracle, T, E, K, shared=256)
    flags = k3x_amd.FLAG_GENERAL_PATH if general else 0
    x = layer.x_bits()
    ref = route_taps(k3x_amd, ctx, cfg, bank, x, flags)
    xb = x.copy()
    xb[1, 77] = {"nan": 0x7FC0, "inf": 0x7F80, "neg_inf": 0xFF80}[bad]
    dev = "cuda:0"
    out = torch.empty((T, cfg.hidden), dtype=torch.int16, device=dev)
    params = k3x_amd.make_params(T, K, cfg.routed_scale, cfg.eps, GLU_SWIGLU, 4.0, None,
                                 RENORM_FLOAT, flags)
    xd = torch.from_numpy(xb.view(np.int16)).to(dev)
    assert k3x_amd.moe_forward(ctx, bank, params, xd, out) == 0
    assert ctx.synchronize() == k3x_amd.ERR_INVALID_MXFP4
    assert ctx.synchronize() == 0  # returned once, then cleared
    again = route_taps(k3x_amd, ctx, cfg, bank, x, flags)
    for k in ref:
        assert np.array_equal(ref[k].view(np.uint8), again[k].view(np.uint8)), k
    bank.close()


@pytest.mark.parametrize("general", [False, True], ids=["decode_path", "general_path"])
def test_nonfinite_bias_rejected(hip, oracle, general):
    """A non-finite correction bias makes the router's adjusted score
    non-finite: K3X_ERR_INVALID_STATE under the float renormalisation
    (runtime/src/routing_policy.cpp:40-58).  A host upload is refused before
    it touches the bank (K3X_ERR_INVALID_EXTENT); a device-side router copy
    is not inspected on the host, so the Top-K kernel latches the error and
    synchronize returns it once."""
    k3x_amd, ctx = hip
    T, E, K = 2, 64, 4
    cfg, layer, bank = small_layer(k3x_amd, ctx, oracle, T, E, K)
    flags = k3x_amd.FLAG_GENERAL_PATH if general else 0
    bias = layer.bias.copy()
    bias[9] = np.inf
    assert bank.upload_router(layer.router, bias, layer.gamma) == k3x_amd.ERR_INVALID_EXTENT
    dev = "cuda:0"
    on_dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
    assert bank.set_router_device(on_dev(layer.router), on_dev(bias), on_dev(layer.gamma)) == 0
    out = torch.empty((T, cfg.hidden), dtype=torch.int16, device=dev)
    params = k3x_amd.make_params(T, K, cfg.routed_scale, cfg.eps, GLU_SWIGLU, 4.0, None,
                                 RENORM_FLOAT, flags)
    xd = torch.from_numpy(layer.x_bits().view(np.int16)).to(dev)
    assert k3x_amd.moe_forward(ctx, bank, params, xd, out) == 0
    assert ctx.synchronize() == k3x_amd.ERR_INVALID_STATE
    assert bank.upload_router(layer.router, layer.bias, layer.gamma) == 0
    got = route_taps(k3x_amd, ctx, cfg, bank, layer.x_bits(), flags)
    _, ids, _ = layer.route(layer.normed(layer.x_bits()))
    assert np.array_equal(got["ids"].view(np.uint32), ids)
    bank.close()
