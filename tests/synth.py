"""Seeded synthetic layers of the five benchmark configurations, regenerated on the
CPU with the oracle's generator (bit-identical to the device fill of
k3x_hip_bank_fill_synthetic), and the CPU reference of the whole layer.

Test helper: the oracle is the checker here, never the thing under test.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import (GLU_SWIGLU, ORDER_CANON, RENORM_FLOAT, SIGMOID_CR, Oracle, bf16_to_f32,
                    round_bf16)

STREAM_GATE_CODES, STREAM_GATE_SCALES = 1, 2
STREAM_UP_CODES, STREAM_UP_SCALES = 3, 4
STREAM_DOWN_CODES, STREAM_DOWN_SCALES = 5, 6
STREAM_ROUTER, STREAM_BIAS = 7, 8
STREAM_SHARED_GATE, STREAM_SHARED_UP, STREAM_SHARED_DOWN = 9, 10, 11
STREAM_INPUT = 12
STREAM_ZIPF_RANK = 13


def sid(kind: int, expert: int = 0) -> int:
    return (kind << 32) | expert


@dataclass
class Config:
    name: str
    tokens: int
    hidden: int
    inter: int
    experts: int
    top_k: int
    shared_inter: int
    scale_lo: int
    scale_hi: int
    routed_scale: float = 1.0
    eps: float = 1e-6
    router_sigma: float = 0.02
    bias_sigma: float = 0.1
    shared_sigma: float = 0.02
    glu: int = GLU_SWIGLU
    beta: float = 4.0
    linear: float | None = None
    renorm: int = RENORM_FLOAT
    seed: int = 0x4B3358
    x_seed: int = 0x5EED
    zipf_b0: float = 0.0   # > 0: bias[e] = b0 * rank(e)^-zipf_s instead of N(0, bias_sigma)
    zipf_s: float = 1.1
    extra: dict = field(default_factory=dict)


# The five benchmark configurations (tiny layer, one expert, decode T=2,
# verification window T=64, prefill T=2048); E8M0 scale ranges and sigmas as
# the benchmark specification gives them, or chosen here where it does not.
CONFIGS = {
    1: Config("c1_tiny", 1, 256, 512, 16, 4, 0, 121, 125),
    2: Config("c2_one_expert", 1, 7168, 2048, 1, 1, 0, 119, 123),
    3: Config("c3_decode", 2, 7168, 2048, 384, 16, 2048, 119, 123, routed_scale=2.5),
    # b0 = 0.45 puts the busiest expert at ~40 of the 64 tokens (calibrated
    # once on this seed; the test asserts the resulting skew).
    4: Config("c4_verify", 64, 7168, 2048, 384, 16, 2048, 119, 123, routed_scale=2.5,
              zipf_b0=0.45),
    5: Config("c5_prefill", 2048, 7168, 2048, 384, 16, 2048, 119, 123, routed_scale=2.5),
}


class SynthLayer:
    """CPU view of a seeded layer; experts are generated on demand."""

    def __init__(self, o: Oracle, cfg: Config):
        self.o, self.cfg = o, cfg
        c = cfg
        key = lambda kind, e=0: o.stream_key(c.seed, sid(kind, e))
        self.router = o.synth_normal(key(STREAM_ROUTER), c.experts * c.hidden,
                                     c.router_sigma).reshape(c.experts, c.hidden)
        if c.zipf_b0 > 0:
            # Zipf(s) over a seeded permutation of the expert ids: rank(e) is
            # the 1-based position of e when a seeded normal draw is sorted.
            u = o.synth_normal(key(STREAM_ZIPF_RANK), c.experts, 1.0)
            rank = np.argsort(np.argsort(u, kind="stable"), kind="stable") + 1
            self.bias = (c.zipf_b0 * rank.astype(np.float64) ** -c.zipf_s).astype(np.float32)
        else:
            self.bias = o.synth_normal(key(STREAM_BIAS), c.experts, c.bias_sigma)
        self.gamma = np.ones(c.hidden, np.float32)
        self.shared = None
        if c.shared_inter:
            S, H = c.shared_inter, c.hidden
            self.shared = (
                o.synth_normal_bf16(key(STREAM_SHARED_GATE), S * H, c.shared_sigma).reshape(S, H),
                o.synth_normal_bf16(key(STREAM_SHARED_UP), S * H, c.shared_sigma).reshape(S, H),
                o.synth_normal_bf16(key(STREAM_SHARED_DOWN), H * S, c.shared_sigma).reshape(H, S),
            )
        self._experts: dict[int, dict] = {}

    def expert(self, e: int) -> dict:
        if e not in self._experts:
            self._experts[e] = self._make_expert(e)
        return self._experts[e]

    def prefetch(self, experts, threads: int = 16) -> None:
        """Generates the given experts ahead of use on `threads` host threads
        (the generator's C calls run without the interpreter lock)."""
        from concurrent.futures import ThreadPoolExecutor
        todo = sorted({int(e) for e in experts} - set(self._experts))
        if not todo:
            return
        with ThreadPoolExecutor(max(1, threads)) as ex:
            for e, d in zip(todo, ex.map(self._make_expert, todo)):
                self._experts[e] = d

    def _make_expert(self, e: int) -> dict:
        o, c = self.o, self.cfg
        key = lambda kind: o.stream_key(c.seed, sid(kind, e))
        n = c.inter * c.hidden
        return dict(
            gate_packed=o.synth_codes(key(STREAM_GATE_CODES), n // 2),
            gate_scales=o.synth_scales(key(STREAM_GATE_SCALES), n // 32, c.scale_lo,
                                       c.scale_hi),
            up_packed=o.synth_codes(key(STREAM_UP_CODES), n // 2),
            up_scales=o.synth_scales(key(STREAM_UP_SCALES), n // 32, c.scale_lo, c.scale_hi),
            down_packed=o.synth_codes(key(STREAM_DOWN_CODES), n // 2),
            down_scales=o.synth_scales(key(STREAM_DOWN_SCALES), n // 32, c.scale_lo, c.scale_hi),
        )

    def x_bits(self) -> np.ndarray:
        c = self.cfg
        return self.o.synth_normal_bf16(self.o.stream_key(c.x_seed, sid(STREAM_INPUT)),
                                        c.tokens * c.hidden, 1.0).reshape(c.tokens, c.hidden)

    # -- the CPU reference of the whole layer (rounding points of the layer
    #    contract: xn, act -> bf16; per-pair outputs and the ordered sum fp32;
    #    final cast bf16) --------------------------------------------------
    def normed(self, x_bits: np.ndarray) -> np.ndarray:
        x = bf16_to_f32(x_bits)
        return np.stack([round_bf16(self.o.rms_norm(x[t], self.gamma, self.cfg.eps, canon=True))
                         for t in range(x.shape[0])])

    def route(self, xn: np.ndarray, bias=None, sigmoid=SIGMOID_CR, order=ORDER_CANON):
        c = self.cfg
        bias = self.bias if bias is None else bias
        T = xn.shape[0]
        logits = np.zeros((T, c.experts), np.float32)
        ids = np.zeros((T, c.top_k), np.uint32)
        w = np.zeros((T, c.top_k), np.float32)
        for t in range(T):
            logits[t] = self.o.router_logits(self.router, xn[t], order)
            st, ids[t], w[t], _ = self.o.route(logits[t], bias, c.top_k, c.renorm,
                                               c.routed_scale, sigmoid)
            assert st == 0, st
        return logits, ids, w

    def pair_outputs(self, xn, ids, tokens=None):
        """act [T][K][I] and y [T][K][H] for the given tokens (default all)."""
        c = self.cfg
        T = xn.shape[0]
        tokens = range(T) if tokens is None else tokens
        act = np.zeros((T, c.top_k, c.inter), np.float32)
        y = np.zeros((T, c.top_k, c.hidden), np.float32)
        for t in tokens:
            for s in range(c.top_k):
                st, act[t, s], y[t, s] = self.o.expert_ffn(
                    xn[t], self.expert(int(ids[t, s])), c.hidden, c.inter, c.glu, c.beta,
                    c.linear, round_act=True)
                assert st == 0, st
        return act, y

    def shared_out(self, xn, tokens=None):
        c = self.cfg
        T = xn.shape[0]
        out = np.zeros((T, c.hidden), np.float32)
        if self.shared is None:
            return out
        for t in (range(T) if tokens is None else tokens):
            out[t] = self.o.shared_ffn(xn[t], *self.shared, glu=c.glu, beta=c.beta,
                                       linear=c.linear, round_act=True)
        return out

    def combine(self, y, w, shared, tokens=None):
        T = y.shape[0]
        out = np.zeros((T, self.cfg.hidden), np.float32)
        for t in (range(T) if tokens is None else tokens):
            out[t] = self.o.ordered_mix(y[t], w[t]) + shared[t]
        return out
