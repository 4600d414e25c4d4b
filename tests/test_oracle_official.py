"""The official K3 MoE FFN (Stable LatentMoE) in the CPU oracle.

* Known answers: every oracle function on the official path reproduces the
  literal values of the reference's own test, tests/cpp/test_official_moe.cpp
  (hidden, route, latent, expert outputs, mixed, routed, shared, combined,
  output at 1e-6, as that test checks them).
* Against the reference compiled in place (oracle/_ref, this container only):
  prepare, route and the whole FFN bit for bit on random layers.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import (GLU_SITU, RENORM_DOUBLE, SIGMOID_REF, ORDER_SEQ, bf16_to_f32,
                    bf16_bits, round_bf16)

EPS = 1.0e-5
BETA, LINEAR = 4.0, 25.0

# tests/cpp/test_official_moe.cpp:48-88: a two-wide layer, two experts of
# 2x2 MXFP4 matrices with block size 2, identity bf16 projections.
KAT = dict(
    residual_norm=[0x3F80, 0x3F80], residual_proj=[0x3F00, 0xBE80], post_norm=[0x3F80, 0x3F00],
    router=[[0x3F80, 0x0000], [0x0000, 0x3F80], [0xBF80, 0x3F80]],
    correction=[0.0, 0.1, -0.05], identity=[[0x3F80, 0x0000], [0x0000, 0x3F80]],
    routed_norm=[0x3F80, 0x3F80],
    experts=[dict(gate=[0x12, 0x21], up=[0x22, 0x31], down=[0x12, 0x21]),
             dict(gate=[0x21, 0x12], up=[0x12, 0x23], down=[0x12, 0x12])],
    prefix=[0.5, -1.0], residual=[1.0, 0.25])


def close(a, b, tol=1e-6):
    return np.allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), rtol=0, atol=tol)


def u16(a):
    return np.asarray(a, dtype=np.uint16)


def test_official_known_answers(oracle):
    k = KAT
    st, hidden = oracle.official_prepare(k["prefix"], k["residual"], u16(k["residual_norm"]),
                                         u16(k["residual_proj"]), u16(k["post_norm"]), EPS)
    assert st == 0 and close(hidden, [1.2578125, -0.32421875])
    # Route: sequential double logits over the bf16 router, float sigmoid,
    # natural Top-2 with the correction, double-sum contributions.
    W = bf16_to_f32(u16(k["router"]))
    logits = oracle.router_logits(W, hidden, ORDER_SEQ)
    st, ids, contrib, _ = oracle.route(logits, k["correction"], 2, RENORM_DOUBLE, 1.0,
                                       SIGMOID_REF)
    assert st == 0 and list(ids) == [0, 1]
    assert close(contrib, [0.6497964859, 0.3502035439])
    # All-equal logits and corrections: lower ids win, equal contributions
    # (test_official_moe.cpp:98-107).
    st, ids0, c0, _ = oracle.route(np.zeros(3, np.float32), np.zeros(3, np.float32), 2,
                                   RENORM_DOUBLE, 1.0, SIGMOID_REF)
    assert st == 0 and list(ids0) == [0, 1] and list(c0) == [0.5, 0.5]
    ident = u16(k["identity"])
    latent = oracle.bf16_matvec_rounded(hidden, ident)
    assert close(latent, [1.2578125, -0.32421875])
    scales = np.array([127, 127], np.uint8)
    ys = []
    for e in k["experts"]:
        g = oracle.mxfp4_matvec(latent, np.uint8(e["gate"]), scales, 2, 2, 2)[1]
        u = oracle.mxfp4_matvec(latent, np.uint8(e["up"]), scales, 2, 2, 2)[1]
        a = oracle.glu(g, u, GLU_SITU, BETA, LINEAR)
        ys.append(round_bf16(oracle.mxfp4_matvec(a, np.uint8(e["down"]), scales, 2, 2, 2)[1]))
    assert close(ys[0], [0.76171875, 0.3984375]) and close(ys[1], [0.81640625, 0.81640625])
    mixed = round_bf16(oracle.ordered_mix(np.stack(ys), contrib))
    assert close(mixed, [0.78125, 0.54296875])
    routed = oracle.bf16_matvec_rounded(oracle.official_norm(mixed, u16(k["routed_norm"]), EPS),
                                        ident)
    assert close(routed, [1.1640625, 0.80859375])
    shared = oracle.official_shared(hidden, ident, ident, ident, GLU_SITU, BETA, LINEAR)
    assert close(shared, [1.1953125, 0.0439453125])
    combined = round_bf16(routed + shared)
    assert close(combined, [2.359375, 0.8515625])
    out = round_bf16(round_bf16(np.float32(k["prefix"])) + combined)
    assert close(out, [2.859375, -0.1484375])


def random_official(oracle, seed, H, L, I, Is, E):
    """A random official layer: bf16-word weights (~N(0, sigma)), MXFP4 experts of
    hidden L, fp32 correction, and one token's prefix and block residual."""
    rng = np.random.default_rng(seed)
    bf = lambda *shape, s=0.05: bf16_bits(rng.standard_normal(shape).astype(np.float32) * s)
    w = dict(residual_norm=bf(H, s=1.0), residual_proj=bf(H, s=0.05), post_norm=bf(H, s=1.0),
             router=bf(E, H, s=0.05), routed_down=bf(L, H, s=0.03), routed_norm=bf(L, s=1.0),
             routed_up=bf(H, L, s=0.03), shared_gate=bf(Is, H, s=0.03),
             shared_up=bf(Is, H, s=0.03), shared_down=bf(H, Is, s=0.03),
             correction=(rng.standard_normal(E) * 0.1).astype(np.float32))
    experts = []
    for e in range(E):
        key = lambda s: oracle.stream_key(seed * 1000 + e, s)
        experts.append(dict(
            gate_packed=oracle.synth_codes(key(1), I * L // 2),
            gate_scales=oracle.synth_scales(key(2), I * L // 32, 121, 125),
            up_packed=oracle.synth_codes(key(3), I * L // 2),
            up_scales=oracle.synth_scales(key(4), I * L // 32, 121, 125),
            down_packed=oracle.synth_codes(key(5), L * I // 2),
            down_scales=oracle.synth_scales(key(6), L * I // 32, 121, 125)))
    prefix = rng.standard_normal(H).astype(np.float32)
    residual = rng.standard_normal(H).astype(np.float32)
    return w, experts, prefix, residual


@pytest.mark.parametrize("shape", [(256, 128, 128, 256, 8, 4), (512, 256, 128, 0, 12, 3)],
                         ids=["shared", "no_shared"])
def test_official_vs_reference(oracle, reflib, shape):
    H, L, I, Is, E, K = shape
    w, experts, prefix, residual = random_official(oracle, 7 + H, H, L, I, max(Is, 32), E)
    if not Is:  # the reference always runs its shared FFN; zero weights give 0
        for k in ("shared_gate", "shared_up", "shared_down"):
            w[k] = np.zeros_like(w[k])
    st, ref = reflib.official_moe(prefix, residual, w, experts, K, EPS, BETA, LINEAR)
    assert st == 0
    st, hidden = oracle.official_prepare(prefix, residual, w["residual_norm"],
                                         w["residual_proj"], w["post_norm"], EPS)
    assert st == 0
    assert np.array_equal(hidden.view(np.uint32), ref["hidden"].view(np.uint32))
    logits = oracle.router_logits(bf16_to_f32(w["router"]), hidden, ORDER_SEQ)
    st, ids, contrib, _ = oracle.route(logits, w["correction"], K, RENORM_DOUBLE, 1.0,
                                       SIGMOID_REF)
    assert st == 0
    assert list(ids) == list(ref["ids"])
    assert np.array_equal(contrib.view(np.uint32), ref["contributions"].view(np.uint32))
    ow = {k: w[k] for k in ("routed_down", "routed_norm", "routed_up", "shared_gate",
                            "shared_up", "shared_down")}
    st, got = oracle.official_ffn(hidden, prefix, ow, [experts[i] for i in ids], contrib, EPS,
                                  GLU_SITU, BETA, LINEAR)
    assert st == 0
    for key in ("latent", "expert_out", "mixed", "routed", "shared", "out"):
        assert np.array_equal(got[key].view(np.uint32), ref[key].view(np.uint32)), key
