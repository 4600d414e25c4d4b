"""ctypes bindings for the CPU checker libraries.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The product path never imports this module.

* ``Oracle`` wraps ``oracle/liboracle.so``, the C restatement of the reference
  path (k3x_oracle.c, every function cites the reference file:line it follows).
* ``RefLib`` wraps ``oracle/_ref/libk3x_ref.so``, the reference's own CPU
  sources compiled in place by ``oracle/Makefile`` (absent unless built).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libk3x_ref.so")

OK, INVALID_EXTENT, INVALID_MXFP4, INVALID_STATE = 0, 9, 15, 16
GLU_SWIGLU, GLU_SITU = 0, 1
RENORM_FLOAT, RENORM_DOUBLE = 0, 1
SIGMOID_REF, SIGMOID_CR = 0, 1
ORDER_SEQ, ORDER_CANON = 0, 1

_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_u16p = C.POINTER(C.c_uint16)
_u32p = C.POINTER(C.c_uint32)
_sz = C.c_size_t


def _p(a: np.ndarray, ptype):
    return a.ctypes.data_as(ptype)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def bf16_to_f32(words: np.ndarray) -> np.ndarray:
    return (np.asarray(words, dtype=np.uint32) << 16).view(np.float32)


def round_bf16(a: np.ndarray) -> np.ndarray:
    """RNE to bf16 kept in float32 (official_moe.cpp:18-26), vectorised."""
    bits = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (bits & 0x7F800000) == 0x7F800000
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    special = np.where((bits & 0x007FFFFF) != 0, bits | 0x00400000, bits)
    special = (special & 0xFFFF0000).astype(np.uint32)
    return np.where(nan, special, rounded).view(np.float32)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    return (round_bf16(a).view(np.uint32) >> 16).astype(np.uint16)


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        L.k3xo_crc32c.restype = C.c_uint32
        L.k3xo_crc32c.argtypes = [_u8p, _sz]
        L.k3xo_crc32c_table.restype = C.c_uint32
        L.k3xo_crc32c_table.argtypes = [_u8p, _sz]
        L.k3xo_fnv1a64.restype = C.c_uint64
        L.k3xo_fnv1a64.argtypes = [C.c_char_p]
        L.k3xo_round_bf16.restype = C.c_float
        L.k3xo_round_bf16.argtypes = [C.c_float]
        L.k3xo_expf_cr.restype = C.c_float
        L.k3xo_expf_cr.argtypes = [C.c_float]
        L.k3xo_sigmoid.restype = C.c_float
        L.k3xo_sigmoid.argtypes = [C.c_float, C.c_int]
        L.k3xo_canon_dot.restype = C.c_double
        L.k3xo_canon_dot.argtypes = [_f32p, _f32p, _sz]
        L.k3xo_decode_mxfp4.argtypes = [_u8p, _sz, _u8p, _sz, _sz, _sz, _sz, _f32p]
        L.k3xo_moe_layer.argtypes = [C.c_void_p, C.c_int, _u32p, _f32p, _f32p]
        L.k3xo_mxfp4_matvec.argtypes = [_f32p, _sz, _u8p, _sz, _u8p, _sz, _sz, _sz, _sz, _f32p]
        L.k3xo_rms_norm.argtypes = [_f32p, _f32p, _f32p, _sz, C.c_float]
        L.k3xo_rms_norm_canon.argtypes = [_f32p, _f32p, _f32p, _sz, C.c_float]
        L.k3xo_glu.argtypes = [_f32p, _f32p, _f32p, _sz, C.c_int, C.c_float, C.c_int, C.c_float]
        L.k3xo_router_logits.argtypes = [_f32p, _f32p, _sz, _sz, C.c_int, _f32p]
        L.k3xo_select.argtypes = [_f32p, _f32p, _sz, _sz, C.c_int, C.c_float, _u32p, _f32p]
        L.k3xo_route.argtypes = [_f32p, _f32p, _sz, _sz, C.c_int, C.c_float, C.c_int,
                                 _u32p, _f32p, _f32p]
        L.k3xo_expert_major_plan.argtypes = [_u32p, _f32p, _sz, _sz, C.POINTER(_sz), _u32p,
                                             _u32p, _u32p, _u32p, _f32p]
        L.k3xo_expert_major_csr.argtypes = [_u32p, _sz, _sz, _sz, _u32p, _u32p, _u32p, _u32p,
                                            _u32p, _u32p, _u32p, _u32p]
        L.k3xo_expert_ffn.argtypes = [_f32p, _sz, _sz, _u8p, _u8p, _u8p, _u8p, _u8p, _u8p,
                                      C.c_int, C.c_float, C.c_int, C.c_float, C.c_int,
                                      _f32p, _f32p]
        L.k3xo_bf16_matvec.argtypes = [_f32p, _u16p, _sz, _sz, _f32p]
        L.k3xo_shared_ffn.argtypes = [_f32p, _sz, _sz, _u16p, _u16p, _u16p, C.c_int,
                                      C.c_float, C.c_int, C.c_float, C.c_int, _f32p]
        L.k3xo_ordered_mix.argtypes = [_f32p, _f32p, _sz, _sz, _f32p]
        L.k3xo_bf16_matvec_rounded.argtypes = [_f32p, _u16p, _sz, _sz, _f32p]
        L.k3xo_official_norm.argtypes = [_f32p, _u16p, _sz, C.c_float, _f32p]
        L.k3xo_official_prepare.argtypes = [_f32p, _f32p, _sz, _u16p, _u16p, _u16p, C.c_float,
                                            _f32p]
        L.k3xo_official_shared.argtypes = [_f32p, _sz, _sz, _u16p, _u16p, _u16p, C.c_int,
                                           C.c_float, C.c_int, C.c_float, _f32p]
        L.k3xo_official_ffn.argtypes = ([_f32p, _f32p, _sz, _sz, _sz, _sz] + [_u16p] * 6 +
                                        [C.POINTER(_u8p), _f32p, _sz, C.c_float, C.c_int,
                                         C.c_float, C.c_int, C.c_float] + [_f32p] * 6)
        L.k3xo_dense_matvec.argtypes = [_f32p, _f32p, _sz, _sz, _f32p]
        L.k3xo_dense_situ_mlp.argtypes = [_f32p, _sz, _sz, _sz, _f32p, _f32p, _f32p, C.c_float,
                                          C.c_int, C.c_float, _f32p, _f32p]
        L.k3xo_resident_layer.argtypes = ([_f32p, _sz, _sz, _sz, _sz] + [_f32p] * 6 +
                                          [C.POINTER(_u8p), _f32p, _sz, C.c_float, C.c_float,
                                           C.c_int, C.c_float, _f32p, _f32p])
        L.k3xo_mix64.restype = C.c_uint64
        L.k3xo_mix64.argtypes = [C.c_uint64]
        L.k3xo_stream_key.restype = C.c_uint64
        L.k3xo_stream_key.argtypes = [C.c_uint64, C.c_uint64]
        L.k3xo_synth_codes.argtypes = [C.c_uint64, _sz, _u8p]
        L.k3xo_synth_scales.argtypes = [C.c_uint64, _sz, C.c_uint32, C.c_uint32, _u8p]
        L.k3xo_synth_normal.argtypes = [C.c_uint64, _sz, C.c_float, _f32p]
        L.k3xo_synth_normal_bf16.argtypes = [C.c_uint64, _sz, C.c_float, _u16p]

    # -- scalar helpers ----------------------------------------------------
    def expf_cr(self, x: float) -> float:
        return self.lib.k3xo_expf_cr(x)

    def sigmoid(self, x: float, mode: int = SIGMOID_CR) -> float:
        return self.lib.k3xo_sigmoid(x, mode)

    # -- MXFP4 -------------------------------------------------------------
    def decode_mxfp4(self, packed, scales, rows, cols, group=32):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        out = np.zeros(rows * cols, np.float32)
        st = self.lib.k3xo_decode_mxfp4(_p(packed, _u8p), packed.size, _p(scales, _u8p),
                                        scales.size, rows, cols, group, _p(out, _f32p))
        return st, out.reshape(rows, cols)

    def mxfp4_matvec(self, x, packed, scales, rows, cols, group=32):
        x = f32(x)
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        out = np.zeros(rows, np.float32)
        st = self.lib.k3xo_mxfp4_matvec(_p(x, _f32p), x.size, _p(packed, _u8p), packed.size,
                                        _p(scales, _u8p), scales.size, rows, cols, group,
                                        _p(out, _f32p))
        return st, out

    # -- element-wise -----------------------------------------------------
    def rms_norm(self, x, w, eps, canon=False):
        x, w = f32(x), f32(w)
        out = np.zeros_like(x)
        fn = self.lib.k3xo_rms_norm_canon if canon else self.lib.k3xo_rms_norm
        fn(_p(out, _f32p), _p(x, _f32p), _p(w, _f32p), x.size, eps)
        return out

    def glu(self, gate, up, kind=GLU_SWIGLU, beta=4.0, linear=None):
        gate, up = f32(gate), f32(up)
        out = np.zeros_like(gate)
        self.lib.k3xo_glu(_p(out, _f32p), _p(gate, _f32p), _p(up, _f32p), gate.size, kind,
                          beta, int(linear is not None), linear or 0.0)
        return out

    # -- router -------------------------------------------------------------
    def canon_dot(self, a, b):
        a, b = f32(a), f32(b)
        return self.lib.k3xo_canon_dot(_p(a, _f32p), _p(b, _f32p), a.size)

    def router_logits(self, W, x, order=ORDER_CANON):
        W, x = f32(W), f32(x)
        E, H = W.shape
        out = np.zeros(E, np.float32)
        self.lib.k3xo_router_logits(_p(W, _f32p), _p(x, _f32p), E, H, order, _p(out, _f32p))
        return out

    def select(self, scores, bias, top_k, renorm=RENORM_FLOAT, routed_scale=1.0):
        scores, bias = f32(scores), f32(bias)
        ids = np.zeros(top_k, np.uint32)
        w = np.zeros(top_k, np.float32)
        st = self.lib.k3xo_select(_p(scores, _f32p), _p(bias, _f32p), scores.size, top_k,
                                  renorm, routed_scale, _p(ids, _u32p), _p(w, _f32p))
        return st, ids, w

    def route(self, logits, bias, top_k, renorm=RENORM_FLOAT, routed_scale=1.0,
              sigmoid=SIGMOID_CR):
        logits, bias = f32(logits), f32(bias)
        E = logits.size
        ids = np.zeros(top_k, np.uint32)
        w = np.zeros(top_k, np.float32)
        scores = np.zeros(E, np.float32)
        st = self.lib.k3xo_route(_p(logits, _f32p), _p(bias, _f32p), E, top_k, renorm,
                                 routed_scale, sigmoid, _p(ids, _u32p), _p(w, _f32p),
                                 _p(scores, _f32p))
        return st, ids, w, scores

    # -- grouping -------------------------------------------------------------
    def expert_major_plan(self, ids, contributions):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        c = f32(contributions)
        T, K = ids.shape
        P = T * K
        n = _sz(0)
        ge = np.zeros(P, np.uint32)
        gs = np.zeros(P + 1, np.uint32)
        at = np.zeros(P, np.uint32)
        asl = np.zeros(P, np.uint32)
        ac = np.zeros(P, np.float32)
        st = self.lib.k3xo_expert_major_plan(_p(ids, _u32p), _p(c, _f32p), T, K, C.byref(n),
                                             _p(ge, _u32p), _p(gs, _u32p), _p(at, _u32p),
                                             _p(asl, _u32p), _p(ac, _f32p))
        g = n.value
        return st, dict(group_expert=ge[:g], group_start=gs[:g + 1], token=at, slot=asl,
                        contribution=ac)

    def expert_major_csr(self, ids, experts):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        T, K = ids.shape
        P = T * K
        counts = np.zeros(experts, np.uint32)
        offsets = np.zeros(experts + 1, np.uint32)
        pt = np.zeros(P, np.uint32)
        ps = np.zeros(P, np.uint32)
        fu = np.zeros(experts, np.uint32)
        na = np.zeros(1, np.uint32)
        aa = np.zeros(experts, np.uint32)
        af = np.zeros(experts, np.uint32)
        st = self.lib.k3xo_expert_major_csr(_p(ids, _u32p), T, K, experts, _p(counts, _u32p),
                                            _p(offsets, _u32p), _p(pt, _u32p), _p(ps, _u32p),
                                            _p(fu, _u32p), _p(na, _u32p), _p(aa, _u32p),
                                            _p(af, _u32p))
        n = int(na[0])
        return st, dict(counts=counts, offsets=offsets, pair_token=pt, pair_slot=ps,
                        first_use=fu, n_active=n, active_ascending=aa[:n],
                        active_first_use=af[:n])

    # -- expert FFN / layer pieces -------------------------------------------
    def expert_ffn(self, x, ex, hidden, inter, glu=GLU_SWIGLU, beta=4.0, linear=None,
                   round_act=True):
        x = f32(x)
        out = np.zeros(hidden, np.float32)
        act = np.zeros(inter, np.float32)
        arrs = [np.ascontiguousarray(ex[k], dtype=np.uint8) for k in
                ("gate_packed", "gate_scales", "up_packed", "up_scales", "down_packed",
                 "down_scales")]
        st = self.lib.k3xo_expert_ffn(_p(x, _f32p), hidden, inter,
                                      *[_p(a, _u8p) for a in arrs], glu, beta,
                                      int(linear is not None), linear or 0.0, int(round_act),
                                      _p(act, _f32p), _p(out, _f32p))
        return st, act, out

    def bf16_matvec(self, x, w_bits):
        x = f32(x)
        w = np.ascontiguousarray(w_bits, dtype=np.uint16)
        rows, cols = w.shape
        out = np.zeros(rows, np.float32)
        self.lib.k3xo_bf16_matvec(_p(x, _f32p), _p(w, _u16p), rows, cols, _p(out, _f32p))
        return out

    def shared_ffn(self, x, gate, up, down, glu=GLU_SWIGLU, beta=4.0, linear=None,
                   round_act=True):
        x = f32(x)
        gate, up, down = (np.ascontiguousarray(a, dtype=np.uint16) for a in (gate, up, down))
        inter, hidden = gate.shape
        out = np.zeros(hidden, np.float32)
        self.lib.k3xo_shared_ffn(_p(x, _f32p), hidden, inter, _p(gate, _u16p), _p(up, _u16p),
                                 _p(down, _u16p), glu, beta, int(linear is not None),
                                 linear or 0.0, int(round_act), _p(out, _f32p))
        return out

    def ordered_mix(self, expert_out, weights):
        y = f32(expert_out)
        w = f32(weights)
        K, width = y.shape
        out = np.zeros(width, np.float32)
        self.lib.k3xo_ordered_mix(_p(y, _f32p), _p(w, _f32p), K, width, _p(out, _f32p))
        return out

    # -- official K3 MoE FFN (official_moe.cpp:39-344) -----------------------
    def bf16_matvec_rounded(self, x, w_bits):
        x = f32(x)
        w = np.ascontiguousarray(w_bits, dtype=np.uint16)
        rows, cols = w.shape
        out = np.zeros(rows, np.float32)
        self.lib.k3xo_bf16_matvec_rounded(_p(x, _f32p), _p(w, _u16p), rows, cols,
                                          _p(out, _f32p))
        return out

    def official_norm(self, x, w_bits, eps):
        x = f32(x)
        w = np.ascontiguousarray(w_bits, dtype=np.uint16)
        out = np.zeros(x.size, np.float32)
        self.lib.k3xo_official_norm(_p(x, _f32p), _p(w, _u16p), x.size, eps, _p(out, _f32p))
        return out

    def official_prepare(self, prefix, residual, residual_norm, residual_proj, post_norm, eps):
        prefix, residual = f32(prefix), f32(residual)
        ws = [np.ascontiguousarray(a, dtype=np.uint16) for a in
              (residual_norm, residual_proj, post_norm)]
        out = np.zeros(prefix.size, np.float32)
        st = self.lib.k3xo_official_prepare(_p(prefix, _f32p), _p(residual, _f32p), prefix.size,
                                            *[_p(a, _u16p) for a in ws], eps, _p(out, _f32p))
        return st, out

    def official_shared(self, x, gate, up, down, glu=GLU_SITU, beta=4.0, linear=25.0):
        x = f32(x)
        gate, up, down = (np.ascontiguousarray(a, dtype=np.uint16) for a in (gate, up, down))
        inter, hidden = gate.shape
        out = np.zeros(hidden, np.float32)
        self.lib.k3xo_official_shared(_p(x, _f32p), hidden, inter, _p(gate, _u16p),
                                      _p(up, _u16p), _p(down, _u16p), glu, beta,
                                      int(linear is not None), linear or 0.0, _p(out, _f32p))
        return out

    def crc32c(self, data) -> int:
        """CRC32C of a bytes-like object (runtime/src/crc32c.cpp:22-28)."""
        a = np.frombuffer(bytes(data), dtype=np.uint8)
        return int(self.lib.k3xo_crc32c(_p(np.ascontiguousarray(a), _u8p), a.size))

    def crc32c_table(self, data) -> int:
        a = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8))
        return int(self.lib.k3xo_crc32c_table(_p(a, _u8p), a.size))

    def fnv1a64(self, name: str) -> int:
        return int(self.lib.k3xo_fnv1a64(name.encode()))

    def official_ffn(self, hidden, prefix, weights, experts, contributions, eps,
                     glu=GLU_SITU, beta=4.0, linear=25.0):
        """One token.  weights: dict of bf16-word arrays routed_down [L][H],
        routed_norm [L], routed_up [H][L], shared_gate/up [Is][H] and
        shared_down [H][Is] (Is may be 0); experts: the routed experts (dicts of
        the six MXFP4 arrays, hidden L) in slot order.  Returns status and a
        dict of latent, expert_out, mixed, routed, shared, out."""
        hidden, prefix = f32(hidden), f32(prefix)
        w = {k: np.ascontiguousarray(v, dtype=np.uint16) for k, v in weights.items()}
        L, H = w["routed_down"].shape
        Is = w["shared_gate"].shape[0] if "shared_gate" in w else 0
        if not Is:
            for k in ("shared_gate", "shared_up", "shared_down"):
                w[k] = np.zeros(1, np.uint16)
        keep = [np.ascontiguousarray(e[k], dtype=np.uint8) for e in experts for k in
                ("gate_packed", "gate_scales", "up_packed", "up_scales", "down_packed",
                 "down_scales")]
        I = experts[0]["gate_packed"].size * 2 // L
        ptrs = (_u8p * len(keep))(*[_p(a, _u8p) for a in keep])
        c = f32(contributions)
        K = c.size
        out = {k: np.zeros(n, np.float32) for k, n in
               (("latent", L), ("expert_out", K * L), ("mixed", L), ("routed", H),
                ("shared", H), ("out", H))}
        st = self.lib.k3xo_official_ffn(
            _p(hidden, _f32p), _p(prefix, _f32p), H, L, I, Is,
            *[_p(w[k], _u16p) for k in ("routed_down", "routed_norm", "routed_up",
                                         "shared_gate", "shared_up", "shared_down")],
            ptrs, _p(c, _f32p), K, eps, glu, beta, int(linear is not None), linear or 0.0,
            *[_p(out[k], _f32p) for k in ("latent", "expert_out", "mixed", "routed",
                                           "shared", "out")])
        out["expert_out"] = out["expert_out"].reshape(K, L)
        return st, out

    # -- fp32 backend operations and the resident latent layer ----------------
    def dense_matvec(self, x, W):
        """y = W x (fp32 W [rows][cols]), sequential double sums."""
        x, W = f32(x), f32(W)
        rows, cols = W.shape
        out = np.zeros(rows, np.float32)
        self.lib.k3xo_dense_matvec(_p(x, _f32p), _p(W, _f32p), rows, cols, _p(out, _f32p))
        return out

    def dense_situ_mlp(self, x, gate, up, down, beta, linear=None):
        """(act, out) of the fp32 SiTU MLP; gate/up [I][H], down [O][I]."""
        x, gate, up, down = f32(x), f32(gate), f32(up), f32(down)
        I, H = gate.shape
        O = down.shape[0]
        act = np.zeros(I, np.float32)
        out = np.zeros(O, np.float32)
        self.lib.k3xo_dense_situ_mlp(_p(x, _f32p), H, I, O, _p(gate, _f32p), _p(up, _f32p),
                                     _p(down, _f32p), beta, int(linear is not None),
                                     linear or 0.0, _p(act, _f32p), _p(out, _f32p))
        return act, out

    def resident_layer(self, x, weights, experts, contributions, eps, beta, linear=None):
        """One token of the resident latent layer.  weights: dict of fp32
        routed_down [L][H], routed_norm [L], routed_up [H][L], shared_gate /
        shared_up [S][H], shared_down [H][S]; experts: dicts of the six MXFP4
        arrays at hidden L, in slot order.  Returns status, mixed [L], out [H]."""
        x = f32(x)
        w = {k: f32(v) for k, v in weights.items()}
        L, H = w["routed_down"].shape
        S = w["shared_gate"].shape[0]
        keep = [np.ascontiguousarray(e[k], dtype=np.uint8) for e in experts for k in
                ("gate_packed", "gate_scales", "up_packed", "up_scales", "down_packed",
                 "down_scales")]
        I = experts[0]["gate_packed"].size * 2 // L
        ptrs = (_u8p * len(keep))(*[_p(a, _u8p) for a in keep])
        c = f32(contributions)
        mixed = np.zeros(L, np.float32)
        out = np.zeros(H, np.float32)
        st = self.lib.k3xo_resident_layer(
            _p(x, _f32p), H, L, I, S,
            *[_p(w[k], _f32p) for k in ("routed_down", "routed_norm", "routed_up",
                                         "shared_gate", "shared_up", "shared_down")],
            ptrs, _p(c, _f32p), c.size, eps, beta, int(linear is not None), linear or 0.0,
            _p(mixed, _f32p), _p(out, _f32p))
        return st, mixed, out

    # -- synthetic inputs -----------------------------------------------------
    def moe_layer(self, x, gamma, eps, router, bias, experts, hidden, inter, top_k,
                  routed_scale=1.0, renorm=RENORM_FLOAT, shared=None, glu=GLU_SWIGLU, beta=4.0,
                  linear=None, round_act=False, threads=1):
        """The whole layer over T tokens as the reference CPU backend composes
        it (k3xo_moe_layer), on `threads` threads.  experts: sequence over all
        expert ids of dicts of the six MXFP4 arrays, or None for experts no
        route reaches; shared: (gate, up, down) bf16-word arrays or None.
        Returns status, ids [T][K], weights [T][K], out [T][H]."""
        x = f32(x)
        T = x.shape[0]
        E = len(experts)
        keep = []
        table = (_u8p * (6 * E))()
        for e, ex in enumerate(experts):
            if ex is None:
                continue
            for k, name in enumerate(("gate_packed", "gate_scales", "up_packed", "up_scales",
                                      "down_packed", "down_scales")):
                a = np.ascontiguousarray(ex[name], dtype=np.uint8)
                keep.append(a)
                table[6 * e + k] = _p(a, _u8p)
        g, r, b = f32(gamma), f32(router), f32(bias)
        sh = [np.ascontiguousarray(m, dtype=np.uint16) for m in shared] if shared else []
        args = _LayerArgs()
        args.x, args.gamma, args.epsilon = _p(x, _f32p), _p(g, _f32p), eps
        args.router, args.bias = _p(r, _f32p), _p(b, _f32p)
        args.tokens, args.hidden, args.inter, args.experts = T, hidden, inter, E
        args.top_k = top_k
        args.shared_inter = sh[0].shape[0] if sh else 0
        args.routed_scale, args.renorm = routed_scale, renorm
        args.expert_bytes = C.cast(table, C.POINTER(_u8p))
        if sh:
            args.shared_gate, args.shared_up, args.shared_down = (_p(m, _u16p) for m in sh)
        args.glu, args.beta = glu, beta
        args.has_linear, args.linear_beta = int(linear is not None), linear or 0.0
        args.round_act = int(round_act)
        ids = np.zeros((T, top_k), np.uint32)
        w = np.zeros((T, top_k), np.float32)
        out = np.zeros((T, hidden), np.float32)
        st = self.lib.k3xo_moe_layer(C.byref(args), threads, _p(ids, _u32p), _p(w, _f32p),
                                     _p(out, _f32p))
        return st, ids, w, out

    def stream_key(self, seed: int, stream: int) -> int:
        return self.lib.k3xo_stream_key(seed, stream)

    def synth_codes(self, key, nbytes):
        out = np.zeros(nbytes, np.uint8)
        self.lib.k3xo_synth_codes(key, nbytes, _p(out, _u8p))
        return out

    def synth_scales(self, key, n, lo, hi):
        out = np.zeros(n, np.uint8)
        self.lib.k3xo_synth_scales(key, n, lo, hi, _p(out, _u8p))
        return out

    def synth_normal(self, key, n, sigma):
        out = np.zeros(n, np.float32)
        self.lib.k3xo_synth_normal(key, n, sigma, _p(out, _f32p))
        return out

    def synth_normal_bf16(self, key, n, sigma):
        out = np.zeros(n, np.uint16)
        self.lib.k3xo_synth_normal_bf16(key, n, sigma, _p(out, _u16p))
        return out


class _LayerArgs(C.Structure):
    _fields_ = [("x", _f32p), ("gamma", _f32p), ("epsilon", C.c_float), ("router", _f32p),
                ("bias", _f32p), ("tokens", _sz), ("hidden", _sz), ("inter", _sz),
                ("experts", _sz), ("top_k", _sz), ("shared_inter", _sz),
                ("routed_scale", C.c_float), ("renorm", C.c_int),
                ("expert_bytes", C.POINTER(_u8p)), ("shared_gate", _u16p),
                ("shared_up", _u16p), ("shared_down", _u16p), ("glu", C.c_int),
                ("beta", C.c_float), ("has_linear", C.c_int), ("linear_beta", C.c_float),
                ("round_act", C.c_int)]


class _ExpertBytes(C.Structure):
    _fields_ = [(n, _u8p) for n in ("gate_packed", "gate_scales", "up_packed", "up_scales",
                                   "down_packed", "down_scales")]


def expert_struct(ex) -> tuple[_ExpertBytes, list]:
    keep = [np.ascontiguousarray(ex[k], dtype=np.uint8) for k in
            ("gate_packed", "gate_scales", "up_packed", "up_scales", "down_packed",
             "down_scales")]
    return _ExpertBytes(*[_p(a, _u8p) for a in keep]), keep


class RefLib:
    """The reference's own CPU path (compiled from its sources by the Makefile)."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.k3xr_crc32c.restype = C.c_uint32
        L.k3xr_crc32c.argtypes = [_u8p, _sz]
        L.k3xr_decode_mxfp4.argtypes = [_u8p, _sz, _u8p, _sz, _sz, _sz, _sz, _f32p]
        L.k3xr_mxfp4_matvec.argtypes = [_f32p, _sz, _u8p, _sz, _u8p, _sz, _sz, _sz, _sz, _f32p]
        L.k3xr_rms_norm.argtypes = [_f32p, _f32p, _f32p, _sz, C.c_float]
        L.k3xr_situ_glu.argtypes = [_f32p, _f32p, _f32p, _sz, C.c_float, C.c_int, C.c_float]
        L.k3xr_route_official_logits.argtypes = [_f32p, _f32p, _sz, _sz, _u32p, _f32p, _f32p]
        L.k3xr_select_routing_natural.argtypes = [_f32p, _f32p, _sz, _sz, _u32p, _f32p]
        L.k3xr_expert_major_plan.argtypes = [_u32p, _f32p, _sz, _sz, C.POINTER(_sz), _u32p,
                                             _u32p, _u32p, _u32p, _f32p]
        L.k3xr_dense_matvec.argtypes = [_f32p, _f32p, _sz, _sz, _f32p]
        EB = C.POINTER(_ExpertBytes)
        L.k3xr_mxfp4_situ_mlp_group.argtypes = [_f32p, _sz, _sz, EB, _sz, C.c_float, C.c_int,
                                                C.c_float, _f32p]
        L.k3xr_mxfp4_situ_moe.argtypes = [_f32p, _sz, _sz, EB, _f32p, _sz, C.c_float, C.c_int,
                                          C.c_float, _f32p]
        L.k3xr_route_tokens.argtypes = [_f32p, _sz, _f32p, C.c_float, _f32p, _f32p, _sz, _sz,
                                        _sz, C.c_float, C.c_int, _u32p, _f32p]
        L.k3xr_official_moe.argtypes = ([_f32p, _f32p] + [_sz] * 6 + [_u16p] * 4 + [_f32p] +
                                        [_u16p] * 6 + [EB, C.c_float, C.c_float, C.c_int,
                                                       C.c_float, _f32p, _u32p] + [_f32p] * 7)
        L.k3xr_moe_layer_token.argtypes = [_f32p, _f32p, C.c_float, _f32p, _f32p, _sz, _sz, _sz,
                                           _sz, C.c_float, EB, _f32p, _f32p, _f32p, _sz,
                                           C.c_float, C.c_int, C.c_float, _u32p, _f32p]
        L.k3xr_dense_situ_mlp.argtypes = [_f32p, _sz, _sz, _sz, _f32p, _f32p, _f32p, C.c_float,
                                          C.c_int, C.c_float, _f32p]
        L.k3xr_resident_layer.argtypes = ([_f32p, _sz, _sz, _sz, _sz] + [_f32p] * 6 +
                                          [EB, _f32p, _sz, C.c_float, C.c_float, C.c_int,
                                           C.c_float, C.POINTER(C.c_int), _f32p])

    def decode_mxfp4(self, packed, scales, rows, cols, group=32):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        out = np.zeros(rows * cols, np.float32)
        st = self.lib.k3xr_decode_mxfp4(_p(packed, _u8p), packed.size, _p(scales, _u8p),
                                        scales.size, rows, cols, group, _p(out, _f32p))
        return st, out.reshape(rows, cols)

    def mxfp4_matvec(self, x, packed, scales, rows, cols, group=32):
        x = f32(x)
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.uint8)
        out = np.zeros(rows, np.float32)
        st = self.lib.k3xr_mxfp4_matvec(_p(x, _f32p), x.size, _p(packed, _u8p), packed.size,
                                        _p(scales, _u8p), scales.size, rows, cols, group,
                                        _p(out, _f32p))
        return st, out

    def rms_norm(self, x, w, eps):
        x, w = f32(x), f32(w)
        out = np.zeros_like(x)
        self.lib.k3xr_rms_norm(_p(out, _f32p), _p(x, _f32p), _p(w, _f32p), x.size, eps)
        return out

    def situ_glu(self, gate, up, beta, linear=None):
        gate, up = f32(gate), f32(up)
        out = np.zeros_like(gate)
        self.lib.k3xr_situ_glu(_p(out, _f32p), _p(gate, _f32p), _p(up, _f32p), gate.size, beta,
                               int(linear is not None), linear or 0.0)
        return out

    def route_official_logits(self, logits, correction, top_k):
        logits, correction = f32(logits), f32(correction)
        E = logits.size
        ids = np.zeros(top_k, np.uint32)
        c = np.zeros(top_k, np.float32)
        s = np.zeros(E, np.float32)
        st = self.lib.k3xr_route_official_logits(_p(logits, _f32p), _p(correction, _f32p), E,
                                                 top_k, _p(ids, _u32p), _p(c, _f32p),
                                                 _p(s, _f32p))
        return st, ids, c, s

    def select_routing(self, scores, bias, top_k):
        scores, bias = f32(scores), f32(bias)
        ids = np.zeros(top_k, np.uint32)
        w = np.zeros(top_k, np.float32)
        st = self.lib.k3xr_select_routing_natural(_p(scores, _f32p), _p(bias, _f32p),
                                                  scores.size, top_k, _p(ids, _u32p),
                                                  _p(w, _f32p))
        return st, ids, w

    def expert_major_plan(self, ids, contributions):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        c = f32(contributions)
        T, K = ids.shape
        P = T * K
        n = _sz(0)
        ge = np.zeros(P, np.uint32)
        gs = np.zeros(P + 1, np.uint32)
        at = np.zeros(P, np.uint32)
        asl = np.zeros(P, np.uint32)
        ac = np.zeros(P, np.float32)
        st = self.lib.k3xr_expert_major_plan(_p(ids, _u32p), _p(c, _f32p), T, K, C.byref(n),
                                             _p(ge, _u32p), _p(gs, _u32p), _p(at, _u32p),
                                             _p(asl, _u32p), _p(ac, _f32p))
        g = n.value
        return st, dict(group_expert=ge[:g], group_start=gs[:g + 1], token=at, slot=asl,
                        contribution=ac)

    def dense_matvec(self, x, W):
        x, W = f32(x), f32(W)
        rows, cols = W.shape
        out = np.zeros(rows, np.float32)
        st = self.lib.k3xr_dense_matvec(_p(x, _f32p), _p(W, _f32p), rows, cols, _p(out, _f32p))
        return st, out

    def dense_situ_mlp(self, x, gate, up, down, beta, linear=None):
        x, gate, up, down = f32(x), f32(gate), f32(up), f32(down)
        I, H = gate.shape
        O = down.shape[0]
        out = np.zeros(O, np.float32)
        st = self.lib.k3xr_dense_situ_mlp(_p(x, _f32p), H, I, O, _p(gate, _f32p), _p(up, _f32p),
                                          _p(down, _f32p), beta, int(linear is not None),
                                          linear or 0.0, _p(out, _f32p))
        return st, out

    def resident_layer(self, x, weights, experts, contributions, eps, beta, linear=None):
        """CpuBackend::resident_mxfp4_moe_layer for one token: status,
        executed, out [H]."""
        x = f32(x)
        w = {k: f32(v) for k, v in weights.items()}
        L, H = w["routed_down"].shape
        S = w["shared_gate"].shape[0]
        I = experts[0]["gate_packed"].size * 2 // L
        structs, keep = zip(*[expert_struct(e) for e in experts])
        arr = (_ExpertBytes * len(structs))(*structs)
        c = f32(contributions)
        executed = C.c_int(0)
        out = np.zeros(H, np.float32)
        st = self.lib.k3xr_resident_layer(
            _p(x, _f32p), H, L, I, S,
            *[_p(w[k], _f32p) for k in ("routed_down", "routed_norm", "routed_up",
                                         "shared_gate", "shared_up", "shared_down")],
            arr, _p(c, _f32p), c.size, eps, beta, int(linear is not None), linear or 0.0,
            C.byref(executed), _p(out, _f32p))
        del keep
        return st, bool(executed.value), out

    def mxfp4_situ_mlp_group(self, x, experts, hidden, inter, beta, linear=None):
        x = f32(x)
        structs, keep = zip(*[expert_struct(e) for e in experts])
        arr = (_ExpertBytes * len(structs))(*structs)
        out = np.zeros((len(structs), hidden), np.float32)
        st = self.lib.k3xr_mxfp4_situ_mlp_group(_p(x, _f32p), hidden, inter, arr, len(structs),
                                                beta, int(linear is not None), linear or 0.0,
                                                _p(out, _f32p))
        del keep
        return st, out

    def route_tokens(self, x, gamma, eps, router, bias, top_k, routed_scale,
                     round_normed=True):
        """ids, weights [T][K] through the reference's routing functions."""
        x, gamma, router, bias = f32(x), f32(gamma), f32(router), f32(bias)
        T, H = x.shape
        E = bias.size
        ids = np.zeros((T, top_k), np.uint32)
        w = np.zeros((T, top_k), np.float32)
        st = self.lib.k3xr_route_tokens(_p(x, _f32p), T, _p(gamma, _f32p), eps,
                                        _p(router, _f32p), _p(bias, _f32p), E, H, top_k,
                                        routed_scale, int(round_normed), _p(ids, _u32p),
                                        _p(w, _f32p))
        return st, ids, w

    def moe_layer_token(self, x, gamma, eps, router, bias, experts_by_id, hidden, inter,
                        top_k, routed_scale, shared=None, beta=4.0, linear=None):
        """One token through the reference CPU composition; experts_by_id is a
        list indexed by expert id (entries for unrouted experts may be None
        only if they are never selected)."""
        x, gamma, router, bias = f32(x), f32(gamma), f32(router), f32(bias)
        E = bias.size
        zero = dict(gate_packed=np.zeros(1, np.uint8), gate_scales=np.zeros(1, np.uint8),
                    up_packed=np.zeros(1, np.uint8), up_scales=np.zeros(1, np.uint8),
                    down_packed=np.zeros(1, np.uint8), down_scales=np.zeros(1, np.uint8))
        structs, keep = zip(*[expert_struct(e if e is not None else zero)
                              for e in experts_by_id])
        arr = (_ExpertBytes * E)(*structs)
        ids = np.zeros(top_k, np.uint32)
        out = np.zeros(hidden, np.float32)
        if shared is not None:
            sg, su, sd = (f32(a) for a in shared)
            s_inter = sg.shape[0]
        else:
            sg = su = sd = np.zeros(1, np.float32)
            s_inter = 0
        st = self.lib.k3xr_moe_layer_token(_p(x, _f32p), _p(gamma, _f32p), eps,
                                           _p(router, _f32p), _p(bias, _f32p), E, hidden, inter,
                                           top_k, routed_scale, arr, _p(sg, _f32p),
                                           _p(su, _f32p), _p(sd, _f32p), s_inter, beta,
                                           int(linear is not None), linear or 0.0,
                                           _p(ids, _u32p), _p(out, _f32p))
        del keep
        return st, ids, out


    def crc32c(self, data) -> int:
        a = np.frombuffer(bytes(data), dtype=np.uint8)
        return int(self.lib.k3xr_crc32c(_p(np.ascontiguousarray(a), _u8p), a.size))

    def official_moe(self, prefix, residual, weights, experts, top_k, eps, beta=4.0,
                     linear=25.0):
        """One token through the reference's prepare, route and official_moe_cpu
        (official_moe.cpp:156-344).  weights: bf16-word arrays residual_norm [H],
        residual_proj [H], post_norm [H], router [E][H], routed_down [L][H],
        routed_norm [L], routed_up [H][L], shared_gate/up [Is][H],
        shared_down [H][Is]; correction fp32 [E]; experts: E expert dicts."""
        prefix, residual = f32(prefix), f32(residual)
        w = {k: np.ascontiguousarray(v, dtype=np.uint16) for k, v in weights.items()
             if k != "correction"}
        corr = f32(weights["correction"])
        E, H = w["router"].shape
        L = w["routed_down"].shape[0]
        Is = w["shared_gate"].shape[0]
        I = experts[0]["gate_packed"].size * 2 // L
        structs, keep = zip(*[expert_struct(e) for e in experts])
        arr = (_ExpertBytes * E)(*structs)
        ids = np.zeros(top_k, np.uint32)
        res = {k: np.zeros(n, np.float32) for k, n in
               (("hidden", H), ("contributions", top_k), ("latent", L),
                ("expert_out", top_k * L), ("mixed", L), ("routed", H), ("shared", H),
                ("out", H))}
        st = self.lib.k3xr_official_moe(
            _p(prefix, _f32p), _p(residual, _f32p), H, L, I, Is, E, top_k,
            *[_p(w[k], _u16p) for k in ("residual_norm", "residual_proj", "post_norm",
                                         "router")],
            _p(corr, _f32p),
            *[_p(w[k], _u16p) for k in ("routed_down", "routed_norm", "routed_up",
                                         "shared_gate", "shared_up", "shared_down")],
            arr, eps, beta, int(linear is not None), linear or 0.0,
            _p(res["hidden"], _f32p), _p(ids, _u32p),
            *[_p(res[k], _f32p) for k in ("contributions", "latent", "expert_out", "mixed",
                                           "routed", "shared", "out")])
        del keep
        res["ids"] = ids
        res["expert_out"] = res["expert_out"].reshape(top_k, L)
        return st, res


@dataclass
class SynthSpec:
    """Seeded synthetic layer description shared by tests and bench."""
    seed: int
    hidden: int
    inter: int
    experts: int
    top_k: int
    shared_inter: int
    scale_lo: int
    scale_hi: int
