"""The oracle against the reference's own known-answer tests.

Every literal below is taken from a test in the reference tree (cited per
test); the oracle must reproduce it.  CPU only.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import (GLU_SITU, GLU_SWIGLU, INVALID_EXTENT, INVALID_MXFP4, INVALID_STATE, OK,
                    ORDER_CANON, ORDER_SEQ, RENORM_DOUBLE, RENORM_FLOAT, SIGMOID_CR,
                    SIGMOID_REF, bf16_to_f32, round_bf16)


# -- RMSNorm ---------------------------------------------------------------
def test_rms_norm_literal_cpp(oracle):
    # tests/cpp/test_ops.cpp:9-13
    out = oracle.rms_norm([3.0, 4.0], [1.0, 2.0], 0.0)
    scale = np.sqrt(np.float32(12.5))
    assert abs(out[0] - 3.0 / scale) <= 1e-6
    assert abs(out[1] - 8.0 / scale) <= 1e-6


@pytest.mark.parametrize("canon", [False, True])
def test_rms_norm_literal_py(oracle, canon):
    # tests/python/test_ops.py:9-11
    out = oracle.rms_norm([3.0, 4.0], [2.0, 0.5], 0.0, canon=canon)
    np.testing.assert_allclose(out, [1.6970563, 0.5656854], atol=1e-6)


# -- GLU --------------------------------------------------------------------
def test_situ_literal_cpp(oracle):
    # tests/cpp/test_ops.cpp:14-17
    out = oracle.glu([-1.0, 2.0], [3.0, 4.0], GLU_SITU, beta=1.0, linear=1.0)
    e0 = math.tanh(-1.0) * (1.0 / (1.0 + math.exp(1.0))) * math.tanh(3.0)
    assert abs(out[0] - e0) <= 1e-6


def test_situ_literal_py(oracle):
    # tests/python/test_ops.py:14-22
    out = oracle.glu([-1.0, 2.0], [3.0, 4.0], GLU_SITU, beta=1.0, linear=1.0)
    np.testing.assert_allclose(out, [-0.20381131, 0.84854317], atol=1e-6)


def test_situ_official_betas_literal(oracle):
    # tests/python/test_moe.py:54-57: 4 tanh(1/4) sigmoid(1) * 25 tanh(1/25)
    out = oracle.glu([1.0], [1.0], GLU_SITU, beta=4.0, linear=25.0)
    want = 4.0 * math.tanh(0.25) / (1.0 + math.exp(-1.0)) * 25.0 * math.tanh(0.04)
    assert abs(out[0] - want) <= 1e-6


# -- MXFP4 ---------------------------------------------------------------------
def test_mxfp4_literal_cpp(oracle):
    # tests/cpp/test_ops.cpp:18-22
    packed = np.zeros(16, np.uint8)
    packed[0] = 0x10
    st, out = oracle.decode_mxfp4(packed, [127], 1, 32)
    assert st == OK and out[0, 0] == 0.0 and out[0, 1] == 0.5


def test_mxfp4_low_nibble_first(oracle):
    # tests/python/test_ops.py:25-29
    st, out = oracle.decode_mxfp4([0x10, 0x32] + [0] * 14, [127], 1, 32)
    assert st == OK
    assert out[0, :4].tolist() == [0.0, 0.5, 1.0, 1.5]


def test_mxfp4_one_scale_per_group(oracle):
    # tests/python/test_ops.py:32-36
    st, out = oracle.decode_mxfp4([0x11] * 32, [127, 128], 1, 64)
    assert st == OK
    assert (out[0, :32] == 0.5).all() and (out[0, 32:] == 1.0).all()


def test_mxfp4_rejects_reserved_scale(oracle):
    # tests/python/test_ops.py:39-41; runtime/src/ops.cpp:46-49
    st, _ = oracle.decode_mxfp4(np.zeros(16, np.uint8), [255], 1, 32)
    assert st == INVALID_MXFP4
    st, _ = oracle.mxfp4_matvec(np.zeros(32), np.zeros(16, np.uint8), [255], 1, 32)
    assert st == INVALID_MXFP4


def test_mxfp4_rejects_bad_contract(oracle):
    # runtime/src/ops.cpp:36-39: cols % group, sizes
    assert oracle.decode_mxfp4(np.zeros(16, np.uint8), [127], 1, 30, 32)[0] == INVALID_MXFP4
    assert oracle.decode_mxfp4(np.zeros(15, np.uint8), [127], 1, 32)[0] == INVALID_MXFP4
    assert oracle.decode_mxfp4(np.zeros(16, np.uint8), [127, 127], 1, 32)[0] == INVALID_MXFP4


def test_mxfp4_matmul_literal_py(oracle):
    # tests/python/test_ops.py:44-53
    st, out = oracle.mxfp4_matvec([2.0, 3.0] + [0.0] * 30, [0x21] + [0] * 15, [127], 1, 32)
    assert st == OK and out.tolist() == [4.0]


def test_mxfp4_matvec_literal_backend(oracle):
    # tests/cpp/test_backend.cpp:112-121
    x = np.zeros(32, np.float32)
    x[1] = 2.0
    packed = np.zeros(16, np.uint8)
    packed[0] = 0x10
    st, out = oracle.mxfp4_matvec(x, packed, [127], 1, 32)
    assert st == OK and out.tolist() == [1.0]


def test_mxfp4_matvec_beyond_one_block_width(oracle):
    # tests/cuda/test_cuda_mxfp4.cu:96-123 (320 columns, packed[128] = 0x21)
    x = np.zeros(320, np.float32)
    x[256], x[257] = 2.0, 3.0
    packed = np.zeros(160, np.uint8)
    packed[128] = 0x21
    st, out = oracle.mxfp4_matvec(x, packed, np.full(10, 127, np.uint8), 1, 320)
    assert st == OK and out.tolist() == [4.0]


# -- dense GEMV (router logits) ---------------------------------------------
@pytest.mark.parametrize("order", [ORDER_SEQ, ORDER_CANON])
def test_router_logits_dense_literal(oracle, order):
    # tests/cpp/test_backend.cpp:100-110 (dense_matvec is the router GEMV)
    W = np.array([[1.0, 2.0, 3.0], [-2.0, 0.25, 4.0]], np.float32)
    out = oracle.router_logits(W, [2.0, -1.0, 0.5], order)
    assert out.tolist() == [1.5, -2.25]


# -- routing -----------------------------------------------------------------
def test_official_route_literal(oracle):
    # tests/cpp/test_official_moe.cpp:85-98
    logits = [1.2578125, -0.32421875, -1.58203125]
    corr = [0.0, 0.1, -0.05]
    for sig in (SIGMOID_REF, SIGMOID_CR):
        st, ids, w, scores = oracle.route(logits, corr, 2, RENORM_DOUBLE, 1.0, sig)
        assert st == OK
        assert ids.tolist() == [0, 1]
        assert abs(w[0] - 0.6497964859) <= 1e-6 and abs(w[1] - 0.3502035439) <= 1e-6


def test_official_route_tie_goes_to_lower_index(oracle):
    # tests/cpp/test_official_moe.cpp:101-109
    st, ids, w, scores = oracle.route([0.0] * 3, [0.0] * 3, 2, RENORM_DOUBLE, 1.0, SIGMOID_REF)
    assert st == OK
    assert ids.tolist() == [0, 1]
    assert scores.tolist() == [0.5, 0.5, 0.5]
    assert w.tolist() == [0.5, 0.5]


def test_official_route_rejections(oracle):
    # tests/cpp/test_official_moe.cpp:110-127
    z = [0.0] * 3
    bad = [0.0, math.inf, 0.0]
    assert oracle.route(bad, z, 2, RENORM_DOUBLE)[0] == INVALID_EXTENT
    assert oracle.route(z, bad, 2, RENORM_DOUBLE)[0] == INVALID_EXTENT
    assert oracle.route(z, z, 0, RENORM_DOUBLE)[0] == INVALID_EXTENT
    assert oracle.route(z, z, 4, RENORM_DOUBLE)[0] == INVALID_EXTENT
    fmax = float(np.finfo(np.float32).max)
    for sig in (SIGMOID_REF, SIGMOID_CR):
        assert oracle.route([-fmax] * 3, z, 2, RENORM_DOUBLE, 1.0, sig)[0] == INVALID_EXTENT


def test_official_route_python_literal(oracle):
    # tests/python/test_official_moe.py:267-304: hidden bf16 bits, identity-like
    # bf16 router, correction -> ids (3, 2, 5) and the literal contributions.
    hidden = bf16_to_f32(np.array([15785, 16020, 16335, 16458], np.uint16))
    W = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1],
                  [-1, 0, 0, 0], [0, -1, 0, 0]], np.float32)
    corr = [0.0, 0.1, 0.2, 0.3, 0.4, 0.5]
    logits = oracle.router_logits(W, hidden, ORDER_SEQ)
    st, ids, w, _ = oracle.route(logits, corr, 3, RENORM_DOUBLE, 1.0, SIGMOID_REF)
    assert st == OK
    assert ids.tolist() == [3, 2, 5]
    np.testing.assert_allclose(w, [0.4317025244, 0.3755553663, 0.1927421242], atol=1e-7)
    assert abs(float(np.sum(w, dtype=np.float64)) - 1.0) <= 1e-7


def test_select_routing_natural_literal(oracle):
    # tests/cpp/test_routing_policy.cpp:30-46
    scores = [0.8, 0.8, 0.4, 0.7, 0.2, 0.1]
    bias = [0.0, 0.0, 0.5, 0.0, 0.0, 0.0]
    st, ids, w = oracle.select(scores, bias, 4, RENORM_FLOAT, 1.0)
    assert st == OK
    assert ids.tolist() == [2, 0, 1, 3]
    want = np.array([0.4, 0.8, 0.8, 0.7], np.float32) / np.float32(2.7)
    np.testing.assert_allclose(w, want, atol=1e-6)


def test_select_routing_rejections(oracle):
    # runtime/src/routing_policy.cpp:40-50 (invalid_state on bad scores / dims)
    assert oracle.select([0.5, 1.5], [0.0, 0.0], 1)[0] == INVALID_STATE
    assert oracle.select([0.5, -0.1], [0.0, 0.0], 1)[0] == INVALID_STATE
    assert oracle.select([0.5, 0.5], [0.0, math.nan], 1)[0] == INVALID_STATE
    assert oracle.select([0.5, 0.5], [0.0, 0.0], 0)[0] == INVALID_STATE
    assert oracle.select([0.0, 0.0], [0.0, 0.0], 1)[0] == INVALID_STATE  # zero mass


def test_router_bias_changes_selection_not_weights(oracle):
    # tests/python/test_moe.py:18-27 (routed_scale 1.0)
    W = np.array([[2.0, 0.0], [1.0, 0.0], [0.0, 0.0]], np.float32)
    logits = oracle.router_logits(W, [1.0, 0.0], ORDER_SEQ)
    st, ids, w, _ = oracle.route(logits, [0.0, 0.0, 0.9], 2, RENORM_FLOAT, 1.0, SIGMOID_REF)
    assert st == OK
    assert ids.tolist() == [2, 0]
    want = np.array([0.5, 0.8807971])
    np.testing.assert_allclose(w, want / want.sum(), atol=1e-6)


def test_routed_scale_multiplies_after_renorm(oracle):
    # runtime/src/model.cpp:1004-1009: contribution = weight * routed_scale
    scores = [0.8, 0.8, 0.4, 0.7, 0.2, 0.1]
    bias = [0.0, 0.0, 0.5, 0.0, 0.0, 0.0]
    _, _, w1 = oracle.select(scores, bias, 4, RENORM_FLOAT, 1.0)
    _, _, w25 = oracle.select(scores, bias, 4, RENORM_FLOAT, 2.5)
    assert (w25 == w1 * np.float32(2.5)).all()


# -- expert-major grouping -------------------------------------------------------
def test_expert_major_first_use_literal(oracle):
    # tests/cpp/test_expert_major.cpp:24-51
    st, plan = oracle.expert_major_plan(np.array([[2, 1], [1, 3]]), [[0.6, 0.4], [0.7, 0.3]])
    assert st == OK
    assert plan["group_expert"].tolist() == [2, 1, 3]
    assert plan["group_start"].tolist() == [0, 1, 3, 4]
    assert plan["token"].tolist() == [0, 0, 1, 1]
    assert plan["slot"].tolist() == [0, 1, 0, 1]
    assert plan["contribution"].tolist() == [np.float32(v) for v in (0.6, 0.4, 0.7, 0.3)]


def test_expert_major_single_slot_literal(oracle):
    # tests/cpp/test_expert_major.cpp:52-62
    st, plan = oracle.expert_major_plan(np.array([[4], [5]]), [[1.0], [1.0]])
    assert st == OK and plan["group_expert"].tolist() == [4, 5]


def test_expert_major_rejections(oracle):
    # tests/cpp/test_expert_major.cpp:68-100
    assert oracle.expert_major_plan(np.array([[1, 1]]), [[0.5, 0.5]])[0] == INVALID_STATE
    assert oracle.expert_major_plan(np.array([[1]]), [[math.nan]])[0] == INVALID_STATE
    assert oracle.expert_major_plan(np.array([[1]]), [[math.inf]])[0] == INVALID_STATE
    assert oracle.expert_major_plan(np.zeros((0, 2), np.uint32), np.zeros((0, 2)))[0] == \
        INVALID_EXTENT


# -- ordered mix --------------------------------------------------------------------
def test_ordered_mix_literal(oracle):
    # tests/cuda/test_cuda_moe_layer_ops.cu:19-24
    y = np.array([[1.0, 2.0, 3.0, 4.0], [-2.0, 1.0, 0.5, 8.0]], np.float32)
    out = oracle.ordered_mix(y, [0.75, -0.25])
    assert out.tolist() == [1.25, 1.25, 2.125, 1.0]


# -- bf16 --------------------------------------------------------------------------
def test_bf16_decode_literals():
    # tests/cpp/test_official_moe.cpp:41-45
    v = bf16_to_f32(np.array([0x0000, 0x8000, 0x3F80, 0x7F80, 0x7FC1], np.uint16))
    assert v[0] == 0.0 and math.copysign(1.0, v[1]) < 0 and v[2] == 1.0
    assert math.isinf(v[3]) and math.isnan(v[4])


# -- the official expert composition --------------------------------------------------
def test_official_expert_outputs_literal(oracle):
    # tests/cpp/test_official_moe.cpp:54-66,129-141: two 2x2 MXFP4 experts
    # (group 2), latent (1.2578125, -0.32421875), SiTU beta 4 / linear 25,
    # down output rounded to bf16 (runtime/src/official_moe.cpp:82-103).
    latent = np.array([1.2578125, -0.32421875], np.float32)
    experts = [
        ([0x12, 0x21], [0x22, 0x31], [0x12, 0x21]),
        ([0x21, 0x12], [0x12, 0x23], [0x12, 0x12]),
    ]
    want = [[0.76171875, 0.3984375], [0.81640625, 0.81640625]]
    outs = []
    for (g, u, d), w in zip(experts, want):
        _, gate = oracle.mxfp4_matvec(latent, g, [127, 127], 2, 2, 2)
        _, up = oracle.mxfp4_matvec(latent, u, [127, 127], 2, 2, 2)
        act = oracle.glu(gate, up, GLU_SITU, 4.0, 25.0)
        st, y = oracle.mxfp4_matvec(act, d, [127, 127], 2, 2, 2)
        y = round_bf16(y)
        assert st == OK
        np.testing.assert_allclose(y, w, atol=1e-6)
        outs.append(y)
    # Slot-ordered mix with the routed contributions, rounded to bf16
    # (mixed_latent literal, test_official_moe.cpp:135).
    mixed = round_bf16(oracle.ordered_mix(np.stack(outs), [0.6497964859, 0.3502035439]))
    np.testing.assert_allclose(mixed, [0.78125, 0.54296875], atol=1e-6)


def test_swiglu_is_silu_times_up(oracle):
    # SwiGLU = silu(g) * u, silu(v) = v * sigmoid(v) (runtime/src/model.cpp:60-61)
    g = np.array([-3.0, -0.5, 0.0, 0.25, 2.0, 9.0], np.float32)
    u = np.array([1.0, -2.0, 3.0, 0.5, -1.5, 0.125], np.float32)
    out = oracle.glu(g, u, GLU_SWIGLU)
    want = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(out, want, rtol=2e-7, atol=1e-12)
