"""The oracle against the reference's own CPU sources, compiled in place into
oracle/_ref/libk3x_ref.so by oracle/Makefile (skipped where that library is
absent).  Wherever the oracle follows the reference's order of operations the
results must be bit-identical.  CPU only.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import (GLU_SITU, OK, ORDER_SEQ, RENORM_DOUBLE, RENORM_FLOAT, SIGMOID_REF,
                    bf16_to_f32)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def rand_expert(rng, H, I, lo=118, hi=126):
    ex = {k: rng.integers(0, 256, H * I // 2, dtype=np.uint8)
          for k in ("gate_packed", "up_packed", "down_packed")}
    ex.update({k: rng.integers(lo, hi + 1, H * I // 32, dtype=np.uint8)
               for k in ("gate_scales", "up_scales", "down_scales")})
    return ex


def test_decode_bitexact(oracle, reflib):
    rng = np.random.default_rng(20)
    packed = rng.integers(0, 256, 64 * 256 // 2, dtype=np.uint8)
    scales = rng.integers(0, 255, 64 * 256 // 32, dtype=np.uint8)
    a = oracle.decode_mxfp4(packed, scales, 64, 256)
    b = reflib.decode_mxfp4(packed, scales, 64, 256)
    assert a[0] == b[0] == OK
    assert np.array_equal(bits(a[1]), bits(b[1]))
    scales[3] = 255
    assert oracle.decode_mxfp4(packed, scales, 64, 256)[0] == \
        reflib.decode_mxfp4(packed, scales, 64, 256)[0] != OK


def test_mxfp4_matvec_bitexact(oracle, reflib):
    rng = np.random.default_rng(21)
    rows, cols = 96, 1024
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    scales = rng.integers(115, 130, rows * cols // 32, dtype=np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    a = oracle.mxfp4_matvec(x, packed, scales, rows, cols)
    b = reflib.mxfp4_matvec(x, packed, scales, rows, cols)
    assert a[0] == b[0] == OK
    assert np.array_equal(bits(a[1]), bits(b[1]))


def test_rms_norm_bitexact(oracle, reflib):
    rng = np.random.default_rng(22)
    for n in (2, 255, 7168):
        x = rng.standard_normal(n).astype(np.float32) * 3
        w = rng.uniform(0.5, 2, n).astype(np.float32)
        assert np.array_equal(bits(oracle.rms_norm(x, w, 1e-6)), bits(reflib.rms_norm(x, w, 1e-6)))


@pytest.mark.parametrize("linear", [None, 25.0])
def test_situ_bitexact(oracle, reflib, linear):
    rng = np.random.default_rng(23)
    g = rng.standard_normal(4096).astype(np.float32) * 4
    u = rng.standard_normal(4096).astype(np.float32) * 4
    a = oracle.glu(g, u, GLU_SITU, 4.0, linear)
    b = reflib.situ_glu(g, u, 4.0, linear)
    assert np.array_equal(bits(a), bits(b))


def test_dense_matvec_is_sequential_router(oracle, reflib):
    rng = np.random.default_rng(24)
    W = rng.standard_normal((384, 7168)).astype(np.float32) * 0.02
    x = rng.standard_normal(7168).astype(np.float32)
    st, want = reflib.dense_matvec(x, W)
    assert st == OK
    assert np.array_equal(bits(oracle.router_logits(W, x, ORDER_SEQ)), bits(want))


def test_select_routing_bitexact(oracle, reflib):
    """FLOAT convention == select_routing (natural), with planted ties."""
    rng = np.random.default_rng(25)
    for trial in range(200):
        E = int(rng.integers(2, 400))
        K = int(rng.integers(1, min(E, 32) + 1))
        if trial % 2:
            scores = rng.choice([0.125, 0.5, 0.625], E).astype(np.float32)
            bias = np.zeros(E, np.float32)
        else:
            scores = rng.uniform(0, 1, E).astype(np.float32)
            bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
        a = oracle.select(scores, bias, K, RENORM_FLOAT, 1.0)
        b = reflib.select_routing(scores, bias, K)
        assert a[0] == OK and b[0] == OK
        assert np.array_equal(a[1], b[1])
        assert np.array_equal(bits(a[2]), bits(b[2]))


def test_route_official_logits_bitexact(oracle, reflib):
    """DOUBLE convention with the libm sigmoid == route_official_moe_logits."""
    rng = np.random.default_rng(26)
    for trial in range(200):
        E = int(rng.integers(2, 400))
        K = int(rng.integers(1, min(E, 32) + 1))
        logits = (rng.standard_normal(E) * (0.0 if trial % 5 == 0 else 2)).astype(np.float32)
        corr = (rng.standard_normal(E) * 0.1).astype(np.float32)
        a = oracle.route(logits, corr, K, RENORM_DOUBLE, 1.0, SIGMOID_REF)
        b = reflib.route_official_logits(logits, corr, K)
        assert a[0] == OK and b[0] == OK
        assert np.array_equal(a[1], b[1])
        assert np.array_equal(bits(a[2]), bits(b[2]))
        assert np.array_equal(bits(a[3]), bits(b[3]))


def test_expert_major_plan_bitexact(oracle, reflib):
    rng = np.random.default_rng(27)
    for trial in range(100):
        E = int(rng.integers(2, 100))
        K = int(rng.integers(1, min(E, 16) + 1))
        T = int(rng.integers(1, 30))
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.uint32)
        w = rng.uniform(0, 1, (T, K)).astype(np.float32)
        a = oracle.expert_major_plan(ids, w)
        b = reflib.expert_major_plan(ids, w)
        assert a[0] == b[0] == OK
        for k in ("group_expert", "group_start", "token", "slot"):
            assert np.array_equal(a[1][k], b[1][k]), k
        assert np.array_equal(bits(a[1]["contribution"]), bits(b[1]["contribution"]))
    dup = np.array([[3, 3]], np.uint32)
    assert oracle.expert_major_plan(dup, [[0.5, 0.5]])[0] == \
        reflib.expert_major_plan(dup, [[0.5, 0.5]])[0] != OK


def test_expert_ffn_bitexact(oracle, reflib):
    """expert_ffn without the activation rounding == mxfp4_situ_mlp_group."""
    rng = np.random.default_rng(28)
    H, I = 512, 256
    experts = [rand_expert(rng, H, I) for _ in range(3)]
    x = rng.standard_normal(H).astype(np.float32)
    st, want = reflib.mxfp4_situ_mlp_group(x, experts, H, I, 4.0, 25.0)
    assert st == OK
    for e, ex in enumerate(experts):
        st, _, y = oracle.expert_ffn(x, ex, H, I, GLU_SITU, 4.0, 25.0, round_act=False)
        assert st == OK
        assert np.array_equal(bits(y), bits(want[e]))


def test_layer_token_bitexact(oracle, reflib):
    """The reference's whole CPU composition of one token (rms_norm, router
    dense_matvec, libm sigmoid, select_routing, mxfp4_situ_moe, dense shared
    expert, add) against the oracle composed the same way."""
    rng = np.random.default_rng(29)
    H, I, E, K, S = 256, 512, 16, 4, 256
    experts = [rand_expert(rng, H, I, 121, 125) for _ in range(E)]
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    gamma = np.ones(H, np.float32)
    bf = lambda r, c: bf16_to_f32(((rng.standard_normal((r, c)) * 0.02).astype(np.float32)
                                   .view(np.uint32) >> 16).astype(np.uint16))
    shared = (bf(S, H), bf(S, H), bf(H, S))
    for t in range(4):
        x = rng.standard_normal(H).astype(np.float32)
        st, ids_ref, out_ref = reflib.moe_layer_token(x, gamma, 1e-6, router, bias, experts, H,
                                                      I, K, 2.5, shared, beta=4.0)
        assert st == OK
        xn = oracle.rms_norm(x, gamma, 1e-6)
        logits = oracle.router_logits(router, xn, ORDER_SEQ)
        st, ids, w, _ = oracle.route(logits, bias, K, RENORM_FLOAT, 2.5, SIGMOID_REF)
        assert st == OK and np.array_equal(ids, ids_ref)
        ys = np.stack([oracle.expert_ffn(xn, experts[int(e)], H, I, GLU_SITU, 4.0, None,
                                         round_act=False)[2] for e in ids])
        mixed = oracle.ordered_mix(ys, w)
        shared_bits = [((m.view(np.uint32) >> 16).astype(np.uint16)) for m in shared]
        sh = oracle.shared_ffn(xn, *shared_bits, glu=GLU_SITU, beta=4.0, linear=None,
                               round_act=False)
        out = (mixed + sh).astype(np.float32)
        assert np.array_equal(bits(out), bits(out_ref))


@pytest.mark.parametrize("threads", [1, 3])
def test_threaded_layer_bitexact(oracle, reflib, threads):
    """k3xo_moe_layer (the bench's CPU baseline: tokens and pairs spread over
    threads) equals the reference's own one-token composition, token by
    token, at any thread count."""
    rng = np.random.default_rng(31)
    H, I, E, K, S, T = 256, 512, 16, 4, 256, 5
    experts = [rand_expert(rng, H, I, 121, 125) for _ in range(E)]
    router = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    gamma = np.ones(H, np.float32)
    words = lambda r, c: ((rng.standard_normal((r, c)) * 0.02).astype(np.float32)
                          .view(np.uint32) >> 16).astype(np.uint16)
    shared_bits = (words(S, H), words(S, H), words(H, S))
    x = rng.standard_normal((T, H)).astype(np.float32)
    st, ids, _, out = oracle.moe_layer(x, gamma, 1e-6, router, bias, experts, H, I, K, 2.5,
                                       RENORM_FLOAT, shared_bits, GLU_SITU, 4.0,
                                       threads=threads)
    assert st == OK
    for t in range(T):
        st, ids_ref, out_ref = reflib.moe_layer_token(
            x[t], gamma, 1e-6, router, bias, experts, H, I, K, 2.5,
            tuple(bf16_to_f32(m) for m in shared_bits), beta=4.0)
        assert st == OK
        assert np.array_equal(ids[t], ids_ref)
        assert np.array_equal(bits(out[t]), bits(out_ref))


def rand_latent_weights(rng, H, L, S):
    """fp32 dense weights of a resident latent layer (routed_norm near 1)."""
    g = lambda *shape: (rng.standard_normal(shape) * 0.05).astype(np.float32)
    return dict(routed_down=g(L, H), routed_norm=rng.uniform(0.5, 1.5, L).astype(np.float32),
                routed_up=g(H, L), shared_gate=g(S, H), shared_up=g(S, H), shared_down=g(H, S))


@pytest.mark.parametrize("linear", [None, 25.0])
def test_dense_situ_mlp_bitexact(oracle, reflib, linear):
    """k3xo_dense_situ_mlp == CpuBackend::dense_situ_mlp."""
    rng = np.random.default_rng(31)
    H, I, O = 384, 256, 320
    x = rng.standard_normal(H).astype(np.float32)
    gate, up = (rng.standard_normal((I, H)) * 0.1).astype(np.float32), \
        (rng.standard_normal((I, H)) * 0.1).astype(np.float32)
    down = (rng.standard_normal((O, I)) * 0.1).astype(np.float32)
    st, want = reflib.dense_situ_mlp(x, gate, up, down, 4.0, linear)
    assert st == OK
    _, got = oracle.dense_situ_mlp(x, gate, up, down, 4.0, linear)
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(oracle.dense_matvec(x, gate)), bits(reflib.dense_matvec(x, gate)[1]))


@pytest.mark.parametrize("linear", [None, 25.0])
def test_resident_layer_bitexact(oracle, reflib, linear):
    """k3xo_resident_layer == CpuBackend::resident_mxfp4_moe_layer (executed
    path) on one token: dense fp32 latent, MXFP4 experts, ordered mix,
    RMSNorm, routed_up and the fp32 shared MLP."""
    rng = np.random.default_rng(32)
    H, L, I, S, K = 512, 256, 256, 384, 3
    w = rand_latent_weights(rng, H, L, S)
    experts = [rand_expert(rng, L, I) for _ in range(K)]
    c = np.array([0.5, 0.3, 0.2], np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    st, executed, want = reflib.resident_layer(x, w, experts, c, 1e-6, 4.0, linear)
    assert st == OK and executed
    st, mixed, got = oracle.resident_layer(x, w, experts, c, 1e-6, 4.0, linear)
    assert st == OK
    assert np.array_equal(bits(got), bits(want))
    assert np.abs(mixed).max() > 0
