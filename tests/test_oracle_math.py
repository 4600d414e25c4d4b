"""The oracle against what mathematics fixes: closed forms, exhaustive
enumeration, brute force on small inputs and independent library routines.

These pin the parts of the oracle that the reference's literal tests leave
open (all 16 x 255 MXFP4 values, the correctly rounded exp of the router
sigmoid, the canonical reduction order, grouping on random routes, the
seeded generator).  CPU only.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import (GLU_SITU, GLU_SWIGLU, INVALID_STATE, OK, ORDER_CANON, ORDER_SEQ,
                    RENORM_DOUBLE, RENORM_FLOAT, bf16_bits, bf16_to_f32, round_bf16)

E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_decode_exhaustive_closed_form(oracle):
    """Every (code, scale) pair: value = (-1)^s * m * 2^(scale-127), in fp32
    (OCP MX E2M1 / E8M0), including -0.0 and overflow to inf."""
    scales = np.arange(255, dtype=np.uint8)
    packed = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8),
                     (255, 2)).reshape(-1)
    st, got = oracle.decode_mxfp4(packed, scales, 255, 32)
    assert st == OK
    with np.errstate(over="ignore"):
        for s in range(255):
            for c in range(32):
                code = c % 16
                mag = E2M1[code & 7]
                want = np.float32(math.ldexp(mag, s - 127))
                if code & 8:
                    want = -want
                assert got[s, c].view(np.uint32) == want.view(np.uint32), (s, code)


def _is_correctly_rounded_exp(x: np.float32, f: np.float32) -> bool:
    import mpmath
    mpmath.mp.prec = 200
    e = mpmath.exp(mpmath.mpf(float(x)))
    if not np.isfinite(f):
        return e > mpmath.mpf(float(np.finfo(np.float32).max))
    if f == 0.0:
        return e < mpmath.mpf(2.0) ** -150
    lo = np.nextafter(f, np.float32(0))
    hi = np.nextafter(f, np.float32(np.inf))
    fm = mpmath.mpf(Fraction(float(f)).numerator) / Fraction(float(f)).denominator
    lom = (fm + mpmath.mpf(float(lo))) / 2
    him = (fm + mpmath.mpf(float(hi))) / 2
    return lom <= e <= him


def test_expf_cr_is_correctly_rounded(oracle):
    """expf_cr(x) is the float nearest to e^x (checked against 200-bit mpmath)
    over the router's input range, the subnormal range and overflow."""
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.uniform(-30, 30, 3000), rng.uniform(-1, 1, 1000), rng.uniform(-104, -87, 300),
        rng.uniform(80, 89, 200), np.array([0.0, -0.0, 1.0, -1.0, 88.72283, 88.7229, -103.9,
                                            1e-8, -1e-8, 0.5, np.log(2.0)]),
    ]).astype(np.float32)
    bad = []
    for x in xs:
        f = np.float32(oracle.expf_cr(float(x)))
        if not _is_correctly_rounded_exp(x, f):
            bad.append((float(x), float(f)))
    assert not bad, bad[:5]


def test_sigmoid_cr_close_to_exact(oracle):
    """1/(1+exp(-x)) with a correctly rounded exp and two float operations:
    three roundings of at most 2^-24 relative each, so within 3 ulp of the
    exact sigmoid (an ulp is 2^-24..2^-23 relative), and monotone."""
    import mpmath
    mpmath.mp.prec = 100
    xs = np.sort(np.random.default_rng(2).uniform(-20, 20, 2000).astype(np.float32))
    prev = -1.0
    for x in xs:
        s = np.float32(oracle.sigmoid(float(x)))
        exact = 1 / (1 + mpmath.exp(-mpmath.mpf(float(x))))
        ulp = float(np.spacing(s))
        assert abs(float(exact) - float(s)) <= 3.0 * ulp
        assert s >= prev
        prev = s


def test_canon_dot_exact_on_integers(oracle):
    """With integer-valued inputs every partial sum is exact in double, so the
    canonical order must give the exact dot product."""
    rng = np.random.default_rng(3)
    for n in (1, 7, 256, 300, 7168):
        a = rng.integers(-100, 100, n).astype(np.float32)
        b = rng.integers(-100, 100, n).astype(np.float32)
        assert oracle.canon_dot(a, b) == float(np.dot(a.astype(np.int64), b.astype(np.int64)))


def test_canon_dot_close_to_fsum(oracle):
    rng = np.random.default_rng(4)
    for n in (512, 2048, 7168):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        exact = math.fsum(float(x) * float(y) for x, y in zip(a, b))
        assert abs(oracle.canon_dot(a, b) - exact) <= 1e-12 * max(1.0, abs(exact))


def test_canon_dot_tree_shape(oracle):
    """The canonical order's shape: 256 lane partials, each summed in index
    order, combined by a balanced pairwise tree.  A cancellation pattern
    planted so that the sequential, left-fold and tree orders give three
    different results checks which one is computed."""
    n = 512
    a = np.zeros(n, np.float32)
    b = np.ones(n, np.float32)
    a[0], a[256] = 2.0 ** 60, 1.0        # partial 0: 2^60 + 1 -> 2^60 (rounds away the 1)
    a[1] = -(2.0 ** 60)                  # partial 1 cancels partial 0 in the first tree level
    a[2] = 1.0                           # partial 2
    # tree: ((p0 + p1) + (p2 + p3)) + ... = (0 + 1) = 1
    assert oracle.canon_dot(a, b) == 1.0
    # sequential order would be 2^60 - 2^60 + 1 + 1 = 2 (index 256 after 0..2)
    seq = 0.0
    for x in a.astype(np.float64):
        seq += x
    assert seq == 2.0


def test_rms_norm_orders_agree_on_exact_sums(oracle):
    x = np.random.default_rng(5).integers(-8, 8, 7168).astype(np.float32)
    w = np.ones(7168, np.float32)
    a = oracle.rms_norm(x, w, 1e-6)
    b = oracle.rms_norm(x, w, 1e-6, canon=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_round_bf16_matches_torch():
    """Round-to-nearest-even agrees with torch's float32 -> bfloat16 cast on
    finite values, ties and overflow."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(6)
    bits = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 2 ** 16, 2000, dtype=np.uint32) << 16) | 0x8000
    x = np.concatenate([bits, ties]).view(np.float32)
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf16_bits(x), want)


def test_select_matches_sorting_brute_force(oracle):
    """Natural Top-K equals a stable sort by (-adjusted score, expert id) with
    planted ties; weights are the scores renormalised over the selection."""
    rng = np.random.default_rng(7)
    for trial in range(300):
        E = int(rng.integers(1, 40))
        K = int(rng.integers(1, E + 1))
        scores = rng.choice([0.25, 0.5, 0.75, 0.125], E).astype(np.float32) \
            if trial % 3 == 0 else rng.uniform(0, 1, E).astype(np.float32)
        bias = rng.choice([0.0, 0.25], E).astype(np.float32)
        adjusted = scores + bias
        order = sorted(range(E), key=lambda e: (-float(adjusted[e]), e))[:K]
        for renorm in (RENORM_FLOAT, RENORM_DOUBLE):
            st, ids, w = oracle.select(scores, bias, K, renorm, 2.5)
            if float(scores[order].astype(np.float64).sum()) == 0.0:
                assert st != OK
                continue
            assert st == OK
            assert ids.tolist() == order
            tot = scores[order].astype(np.float64).sum()
            np.testing.assert_allclose(w, scores[order] / tot * 2.5, rtol=3e-7)


def test_expert_major_csr_matches_plan_and_argsort(oracle):
    """The CSR form groups every (token, slot) pair under its expert in
    (token, slot) order, and ordering experts by first use reproduces the
    group order of the plan."""
    rng = np.random.default_rng(8)
    for trial in range(100):
        E = int(rng.integers(2, 64))
        K = int(rng.integers(1, min(E, 16) + 1))
        T = int(rng.integers(1, 40))
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.uint32)
        w = rng.uniform(0.1, 1, (T, K)).astype(np.float32)
        st, csr = oracle.expert_major_csr(ids, E)
        assert st == OK
        flat = ids.reshape(-1)
        perm = np.argsort(flat, kind="stable")
        assert np.array_equal(csr["pair_token"], perm // K)
        assert np.array_equal(csr["pair_slot"], perm % K)
        assert np.array_equal(csr["counts"], np.bincount(flat, minlength=E))
        assert np.array_equal(csr["offsets"][1:], np.cumsum(csr["counts"]))
        st, plan = oracle.expert_major_plan(ids, w)
        assert st == OK
        assert np.array_equal(plan["group_expert"], csr["active_first_use"])
        first = {}
        for p, e in enumerate(flat):
            first.setdefault(int(e), p)
        assert [e for e, _ in sorted(first.items(), key=lambda kv: kv[1])] == \
            plan["group_expert"].tolist()


def test_expert_major_csr_rejects_out_of_range(oracle):
    st, _ = oracle.expert_major_csr(np.array([[0, 5]], np.uint32), 5)
    assert st == INVALID_STATE


def test_expert_major_csr_rejects_what_the_plan_rejects(oracle):
    # One expert twice in one token: the plan's rejection
    # (tests/cpp/test_expert_major.cpp:68-100); the CSR form agrees, and the
    # same expert in two different tokens stays valid.
    ids = np.array([[3, 1], [1, 3]], np.uint32)
    assert oracle.expert_major_csr(ids, 4)[0] == 0
    dup = np.array([[3, 1], [2, 2]], np.uint32)
    assert oracle.expert_major_csr(dup, 4)[0] == INVALID_STATE
    assert oracle.expert_major_plan(dup, np.full((2, 2), 0.5))[0] == INVALID_STATE


def test_splitmix64_known_answer(oracle):
    """The generator's word i of key k is SplitMix64's output i after seeding
    with k (Steele, Lea & Flood 2014): mix(k + (i+1) * golden).  Published
    outputs for seed 1234567."""
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    got = oracle.synth_codes(1234567, 40).view("<u8").tolist()
    assert got == want


def test_synth_normal_moments(oracle):
    """The Irwin-Hall(12) normal has mean 0 and variance sigma^2."""
    x = oracle.synth_normal(oracle.stream_key(42, 7), 200000, 0.5).astype(np.float64)
    assert abs(x.mean()) < 0.005 and abs(x.std() - 0.5) < 0.005
    assert np.abs(x).max() <= 6 * 0.5


def test_synth_scales_uniform(oracle):
    s = oracle.synth_scales(oracle.stream_key(1, 2), 100000, 119, 123)
    counts = np.bincount(s, minlength=256)[119:124]
    assert s.min() == 119 and s.max() == 123
    assert np.all(np.abs(counts / 100000 - 0.2) < 0.01)


def test_mxfp4_matvec_matches_decoded_float64(oracle):
    """GEMV = double-precision dot of the decoded matrix, cast once."""
    rng = np.random.default_rng(9)
    rows, cols = 16, 512
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    scales = rng.integers(118, 126, rows * cols // 32, dtype=np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    st, W = oracle.decode_mxfp4(packed, scales, rows, cols)
    st2, y = oracle.mxfp4_matvec(x, packed, scales, rows, cols)
    assert st == st2 == OK
    exact = [math.fsum(float(a) * float(b) for a, b in zip(W[r], x)) for r in range(rows)]
    np.testing.assert_allclose(y, exact, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("glu", [GLU_SWIGLU, GLU_SITU])
def test_expert_ffn_composition(oracle, glu):
    """expert_ffn = down(round_bf16(GLU(gate x, up x))) composed from the
    decoded matrices in float64."""
    rng = np.random.default_rng(10)
    H, I = 256, 128
    ex = {k: rng.integers(0, 256, H * I // 2, dtype=np.uint8)
          for k in ("gate_packed", "up_packed", "down_packed")}
    ex.update({k: rng.integers(119, 124, H * I // 32, dtype=np.uint8)
               for k in ("gate_scales", "up_scales", "down_scales")})
    x = rng.standard_normal(H).astype(np.float32)
    st, act, y = oracle.expert_ffn(x, ex, H, I, glu, 4.0, 25.0 if glu == GLU_SITU else None)
    assert st == OK
    _, G = oracle.decode_mxfp4(ex["gate_packed"], ex["gate_scales"], I, H)
    _, U = oracle.decode_mxfp4(ex["up_packed"], ex["up_scales"], I, H)
    _, D = oracle.decode_mxfp4(ex["down_packed"], ex["down_scales"], H, I)
    g = (G.astype(np.float64) @ x).astype(np.float32)
    u = (U.astype(np.float64) @ x).astype(np.float32)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    sig = 1 / (1 + np.exp(-gd))
    if glu == GLU_SITU:
        a = 4 * np.tanh(gd / 4) * sig * 25 * np.tanh(ud / 25)
    else:
        a = gd * sig * ud
    np.testing.assert_allclose(act, a, rtol=8e-3, atol=1e-6)  # act is bf16-rounded
    want = D.astype(np.float64) @ act.astype(np.float64)
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-6)


def test_shared_ffn_composition(oracle):
    rng = np.random.default_rng(11)
    H, S = 256, 128
    mk = lambda r, c: bf16_bits(rng.standard_normal((r, c)).astype(np.float32) * 0.05)
    g, u, d = mk(S, H), mk(S, H), mk(H, S)
    x = rng.standard_normal(H).astype(np.float32)
    out = oracle.shared_ffn(x, g, u, d)
    gv = bf16_to_f32(g).astype(np.float64) @ x
    uv = bf16_to_f32(u).astype(np.float64) @ x
    gv, uv = gv.astype(np.float32).astype(np.float64), uv.astype(np.float32).astype(np.float64)
    a = round_bf16((gv / (1 + np.exp(-gv)) * uv).astype(np.float32))
    want = bf16_to_f32(d).astype(np.float64) @ a.astype(np.float64)
    np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-7)
