"""ctypes binding of libk3x_hip_moe.so (the C ABI in include/k3x_hip_moe.h).

torch is used only for device memory and the stream: tensors are passed to
the library as raw device pointers.  There is no fallback: if the HIP library
is missing, or no GPU is present, construction raises.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref
from dataclasses import dataclass

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libk3x_hip_moe.so")

OK = 0
ERR_INVALID_EXTENT = 9
ERR_TENSOR_NOT_FOUND = 14
ERR_INVALID_MXFP4 = 15
ERR_INVALID_STATE = 16
ERR_BACKEND_UNAVAILABLE = 17

GLU_SWIGLU, GLU_SITU = 0, 1
STAGES = ("route", "group", "gate_up", "shared_gate_up", "down", "shared_down", "combine",
          "decode_front", "decode_select", "decode_gate_up", "decode_down")
RENORM_FLOAT, RENORM_DOUBLE = 0, 1
MATRIX_GATE, MATRIX_UP, MATRIX_DOWN = 0, 1, 2

STREAM_GATE_CODES = 1
STREAM_GATE_SCALES = 2
STREAM_UP_CODES = 3
STREAM_UP_SCALES = 4
STREAM_DOWN_CODES = 5
STREAM_DOWN_SCALES = 6
STREAM_ROUTER = 7
STREAM_BIAS = 8
STREAM_SHARED_GATE = 9
STREAM_SHARED_UP = 10
STREAM_SHARED_DOWN = 11
STREAM_INPUT = 12


def stream_id(kind: int, expert: int = 0) -> int:
    return (kind << 32) | expert


class K3xError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what} failed: status {status} ({_name(status)})")


def _name(status: int) -> str:
    return {0: "OK", 9: "INVALID_EXTENT", 14: "TENSOR_NOT_FOUND", 15: "INVALID_MXFP4",
            16: "INVALID_STATE", 17: "BACKEND_UNAVAILABLE"}.get(status, "UNKNOWN")


class LayerDesc(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("inter", C.c_uint32), ("experts", C.c_uint32),
                ("group_size", C.c_uint32), ("shared_inter", C.c_uint32)]


class MoeParams(C.Structure):
    _fields_ = [("tokens", C.c_uint32), ("top_k", C.c_uint32), ("routed_scale", C.c_float),
                ("rms_epsilon", C.c_float), ("glu", C.c_uint32), ("situ_beta", C.c_float),
                ("has_situ_linear", C.c_uint32), ("situ_linear_beta", C.c_float),
                ("renorm", C.c_uint32), ("flags", C.c_uint32)]

FLAG_GENERAL_PATH = 1
FLAG_ROUND_EXPERT_OUT = 2
FLAG_SPLIT_ACT = 4
FLAG_SPLIT_INPUT = 8
FLAG_SCALED_FP4 = 16


class LatentWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("routed_down", "routed_norm", "routed_up",
                                         "shared_gate", "shared_up", "shared_down")] + \
               [("hidden", C.c_uint32), ("latent", C.c_uint32), ("shared_inter", C.c_uint32),
                ("latent_norm", C.c_uint32)]


TAP_FIELDS = ["normed_x", "logits", "ids", "weights", "counts", "offsets", "pair_token",
              "pair_slot", "first_use", "n_active", "active_first_use", "act", "expert_out",
              "shared_out", "out_f32", "shared_act"]


class MoeTaps(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in TAP_FIELDS]


OFFICIAL_TAP_FIELDS = ["logits", "ids", "contributions", "latent", "expert_out", "mixed",
                       "routed", "shared"]


class OfficialTaps(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in OFFICIAL_TAP_FIELDS]


class OfficialDesc(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("shared_inter", C.c_uint32),
                ("router_experts", C.c_uint32)]


class SynthDesc(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("scale_lo", C.c_uint32), ("scale_hi", C.c_uint32),
                ("router_sigma", C.c_float), ("bias_sigma", C.c_float),
                ("shared_sigma", C.c_float), ("gamma_value", C.c_float)]


class Stats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("forward_calls", "kernel_launches", "scratch_bytes",
                                         "resident_weight_bytes", "weight_h2d_bytes",
                                         "experts_resident")]


_vp = C.c_void_p
_LIB = None

# name -> (restype, argtypes)
_SIGS = {
    "k3x_hip_status_name": (C.c_char_p, [C.c_int]),
    "k3x_hip_ctx_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "k3x_hip_ctx_destroy": (C.c_int, [_vp]),
    "k3x_hip_ctx_set_stream": (C.c_int, [_vp, _vp]),
    "k3x_hip_ctx_use_own_stream": (C.c_int, [_vp]),
    "k3x_hip_ctx_stream": (_vp, [_vp]),
    "k3x_hip_ctx_synchronize": (C.c_int, [_vp]),
    "k3x_hip_ctx_stats": (C.c_int, [_vp, C.POINTER(Stats)]),
    "k3x_hip_ctx_set_profiling": (C.c_int, [_vp, C.c_int]),
    "k3x_hip_ctx_stage_times": (C.c_int, [_vp, C.POINTER(C.c_double), C.POINTER(C.c_uint64),
                                          C.c_int]),
    "k3x_hip_bank_create": (C.c_int, [_vp, C.POINTER(LayerDesc), C.POINTER(_vp)]),
    "k3x_hip_bank_destroy": (C.c_int, [_vp]),
    "k3x_hip_bank_upload_expert": (C.c_int, [_vp, C.c_uint32, C.POINTER(C.c_uint64), _vp, _vp,
                                             _vp, _vp, _vp, _vp]),
    "k3x_hip_crc32c": (C.c_int, [_vp, _vp, C.c_size_t, C.POINTER(C.c_uint32)]),
    "k3x_hip_stream_read": (C.c_int, [_vp, _vp, C.c_size_t, _vp]),
    "k3x_hip_storage_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "k3x_hip_storage_close": (C.c_int, [_vp]),
    "k3x_hip_storage_upload_expert": (C.c_int, [_vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32,
                                                C.POINTER(C.c_uint64), C.c_void_p]),
    "k3x_hip_storage_verify": (C.c_int, [_vp]),
    "k3x_hip_bank_upload_expert_device": (C.c_int, [_vp, C.c_uint32, C.POINTER(C.c_uint64),
                                                    C.POINTER(_vp), C.POINTER(C.c_uint32)]),
    "k3x_hip_bank_find": (C.c_int, [_vp, C.c_uint64, C.POINTER(C.c_uint32),
                                    C.POINTER(C.c_uint32)]),
    "k3x_hip_bank_upload_shared": (C.c_int, [_vp, _vp, _vp, _vp]),
    "k3x_hip_bank_upload_router": (C.c_int, [_vp, _vp, _vp, _vp]),
    "k3x_hip_bank_set_router_device": (C.c_int, [_vp, _vp, _vp, _vp]),
    "k3x_hip_bank_fill_synthetic": (C.c_int, [_vp, C.POINTER(SynthDesc)]),
    "k3x_hip_synth_normal_bf16": (C.c_int, [_vp, C.c_uint64, C.c_uint64, C.c_float, C.c_size_t,
                                            _vp]),
    "k3x_hip_bank_dequant_rows": (C.c_int, [_vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                            _vp]),
    "k3x_hip_bank_bytes": (C.c_uint64, [_vp]),
    "k3x_hip_moe_forward": (C.c_int, [_vp, _vp, C.POINTER(MoeParams), _vp, _vp,
                                      C.POINTER(MoeTaps)]),
    "k3x_hip_moe_forward_noalloc": (C.c_int, [_vp, _vp, C.POINTER(MoeParams), _vp, _vp,
                                              C.POINTER(MoeTaps)]),
    "k3x_hip_moe_forward_routed": (C.c_int, [_vp, _vp, C.POINTER(MoeParams), _vp, _vp, _vp, _vp,
                                             _vp, _vp, C.POINTER(MoeTaps)]),
    "k3x_hip_expert_major_plan": (C.c_int, [_vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32,
                                            C.POINTER(MoeTaps)]),
    "k3x_hip_official_create": (C.c_int, [_vp, _vp, C.POINTER(OfficialDesc), C.POINTER(_vp)]),
    "k3x_hip_official_destroy": (C.c_int, [_vp]),
    "k3x_hip_official_upload_ffn": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "k3x_hip_official_upload_route": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "k3x_hip_official_fill_synthetic": (C.c_int, [_vp, C.c_uint64, C.c_float, C.c_float,
                                                  C.c_float, C.c_float]),
    "k3x_hip_official_prepare": (C.c_int, [_vp, _vp, C.c_uint32, C.c_float, _vp, _vp, _vp, _vp]),
    "k3x_hip_official_ffn": (C.c_int, [_vp, _vp, C.POINTER(MoeParams), _vp, _vp, _vp, _vp, _vp,
                                       C.POINTER(OfficialTaps)]),
    "k3x_hip_dense_f32_matvec": (C.c_int, [_vp, _vp, C.c_uint32, C.c_uint32, _vp, C.c_uint32,
                                           _vp]),
    "k3x_hip_mxfp4_matvec": (C.c_int, [_vp, _vp, _vp, C.c_uint32, C.c_uint32, _vp, C.c_uint32,
                                       _vp]),
    "k3x_hip_dense_situ_mlp": (C.c_int, [_vp, _vp, _vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32,
                                         C.c_float, C.c_int, C.c_float, _vp, C.c_uint32, _vp,
                                         _vp]),
    "k3x_hip_resident_moe_layer": (C.c_int, [_vp, _vp, C.POINTER(LatentWeights),
                                             C.POINTER(MoeParams), _vp, _vp, _vp, _vp, _vp, _vp,
                                             _vp]),
}

EXPORTED = sorted(_SIGS)


def load(path: str = LIB_PATH) -> C.CDLL:
    """Loads the HIP library and declares every entry point; raises if absent."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: build it with `make -C project-k3x_amd` "
                "(or __graft_entry__.build())")
        lib = C.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def check(status: int, what: str) -> None:
    if status != OK:
        raise K3xError(status, what)


def ptr(t) -> int | None:
    """Device pointer of a torch tensor (None passes through)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t.data_ptr()


def host_ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Context:
    def __init__(self, device: int = 0, use_torch_stream: bool = True):
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("no HIP device: the MoE layer has no CPU path")
        self.lib = load()
        h = _vp()
        check(self.lib.k3x_hip_ctx_create(device, C.byref(h)), "k3x_hip_ctx_create")
        self.handle = h
        self.device = device
        self._banks = weakref.WeakSet()
        if use_torch_stream:
            with torch.cuda.device(device):
                s = torch.cuda.current_stream().cuda_stream
            check(self.lib.k3x_hip_ctx_set_stream(h, _vp(s)), "k3x_hip_ctx_set_stream")

    def synchronize(self) -> int:
        return self.lib.k3x_hip_ctx_synchronize(self.handle)

    def crc32c(self, data, nbytes: int | None = None) -> tuple[int, int]:
        """(status, CRC32C) of a device tensor's bytes (k3x_hip_crc32c)."""
        n = data.numel() * data.element_size() if nbytes is None else nbytes
        out = C.c_uint32(0)
        st = self.lib.k3x_hip_crc32c(self.handle, ptr(data), n, C.byref(out))
        return st, out.value

    def stream_read(self, data, fold, nbytes: int | None = None) -> int:
        """Enqueues k3x_hip_stream_read over a device tensor's bytes, XOR-folding
        its 32-bit words into the device dword `fold`."""
        n = data.numel() * data.element_size() if nbytes is None else nbytes
        return self.lib.k3x_hip_stream_read(self.handle, ptr(data), n, ptr(fold))

    def stats(self) -> Stats:
        s = Stats()
        check(self.lib.k3x_hip_ctx_stats(self.handle, C.byref(s)), "k3x_hip_ctx_stats")
        return s

    def set_profiling(self, enabled: bool) -> None:
        check(self.lib.k3x_hip_ctx_set_profiling(self.handle, int(enabled)),
              "k3x_hip_ctx_set_profiling")

    def stage_times(self, reset: bool = True) -> dict:
        """{stage: (total_ms, launches)} since the last reset (synchronises)."""
        n = len(STAGES)
        ms = (C.c_double * n)()
        cnt = (C.c_uint64 * n)()
        check(self.lib.k3x_hip_ctx_stage_times(self.handle, ms, cnt, int(reset)),
              "k3x_hip_ctx_stage_times")
        return {name: (ms[i], cnt[i]) for i, name in enumerate(STAGES)}

    def close(self) -> None:
        """Destroys the context after every bank created on it."""
        if self.handle:
            for off in list(getattr(self, "_officials", ())):
                off.close()
            for bank in list(self._banks):
                bank.close()
            check(self.lib.k3x_hip_ctx_destroy(self.handle), "k3x_hip_ctx_destroy")
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class LayerShape:
    hidden: int
    inter: int
    experts: int
    shared_inter: int = 0
    group_size: int = 32

    def desc(self) -> LayerDesc:
        return LayerDesc(self.hidden, self.inter, self.experts, self.group_size,
                         self.shared_inter)

    def routed_bytes_per_expert(self) -> int:
        n = self.hidden * self.inter
        return 3 * (n // 2 + n // 32)


class Bank:
    def __init__(self, ctx: Context, shape: LayerShape):
        self.ctx = ctx
        self.lib = ctx.lib
        self.shape = shape
        h = _vp()
        d = shape.desc()
        check(self.lib.k3x_hip_bank_create(ctx.handle, C.byref(d), C.byref(h)),
              "k3x_hip_bank_create")
        self.handle = h
        ctx._banks.add(self)

    def fill_synthetic(self, seed: int, scale_lo: int, scale_hi: int, router_sigma=0.02,
                       bias_sigma=0.1, shared_sigma=0.02, gamma=1.0) -> None:
        d = SynthDesc(seed, scale_lo, scale_hi, router_sigma, bias_sigma, shared_sigma, gamma)
        check(self.lib.k3x_hip_bank_fill_synthetic(self.handle, C.byref(d)),
              "k3x_hip_bank_fill_synthetic")

    def upload_expert(self, expert: int, ex: dict, tensor_ids=None) -> int:
        import numpy as np
        ids = tensor_ids or (3 * expert + 1, 3 * expert + 2, 3 * expert + 3)
        arr = (C.c_uint64 * 3)(*ids)
        keep = [np.ascontiguousarray(ex[k], dtype=np.uint8) for k in
                ("gate_packed", "gate_scales", "up_packed", "up_scales", "down_packed",
                 "down_scales")]
        return self.lib.k3x_hip_bank_upload_expert(self.handle, expert, arr,
                                                   *[host_ptr(a) for a in keep])

    def upload_expert_device(self, expert: int, extents, tensor_ids, crcs=None) -> int:
        """Six device extents (gate codes, gate scales, up codes, up scales,
        down codes, down scales), checked against crcs (six CRC32C values)."""
        ids = (C.c_uint64 * 3)(*tensor_ids)
        ptrs = (_vp * 6)(*[ptr(e) for e in extents])
        c = (C.c_uint32 * 6)(*crcs) if crcs is not None else None
        return self.lib.k3x_hip_bank_upload_expert_device(self.handle, expert, ids, ptrs, c)

    def upload_shared(self, gate, up, down) -> int:
        import numpy as np
        g, u, d = (np.ascontiguousarray(a, dtype=np.uint16) for a in (gate, up, down))
        return self.lib.k3x_hip_bank_upload_shared(self.handle, host_ptr(g), host_ptr(u),
                                                   host_ptr(d))

    def upload_router(self, weight, bias, gamma) -> int:
        import numpy as np
        w, b, g = (np.ascontiguousarray(a, dtype=np.float32) for a in (weight, bias, gamma))
        return self.lib.k3x_hip_bank_upload_router(self.handle, host_ptr(w), host_ptr(b),
                                                   host_ptr(g))

    def set_router_device(self, weight, bias, gamma) -> int:
        """Router weights [E][H], bias [E], gamma [H] from fp32 device tensors
        (queued on the context stream)."""
        return self.lib.k3x_hip_bank_set_router_device(self.handle, ptr(weight), ptr(bias),
                                                       ptr(gamma))

    def find(self, tensor_id: int):
        e, m = C.c_uint32(0), C.c_uint32(0)
        st = self.lib.k3x_hip_bank_find(self.handle, tensor_id, C.byref(e), C.byref(m))
        return st, e.value, m.value

    def dequant_rows(self, expert: int, matrix: int, row0: int, nrows: int):
        import torch
        cols = self.shape.hidden if matrix != MATRIX_DOWN else self.shape.inter
        out = torch.empty((nrows, cols), dtype=torch.float32, device=f"cuda:{self.ctx.device}")
        check(self.lib.k3x_hip_bank_dequant_rows(self.handle, expert, matrix, row0, nrows,
                                                 ptr(out)), "k3x_hip_bank_dequant_rows")
        return out

    def bytes(self) -> int:
        return self.lib.k3x_hip_bank_bytes(self.handle)

    def close(self) -> None:
        if self.handle:
            self.lib.k3x_hip_bank_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Official:
    """The official K3 MoE FFN around a bank of experts at the latent width
    (k3x_hip_official_*); host weights are bf16 words (uint16 numpy arrays)."""

    def __init__(self, ctx: Context, experts: Bank | None, hidden: int, shared_inter: int,
                 router_experts: int = 0):
        """experts None: a route-only object (upload_route, fill_synthetic,
        prepare) whose router has router_experts rows."""
        import weakref
        self.ctx, self.lib, self.experts = ctx, ctx.lib, experts
        self.hidden, self.shared_inter = hidden, shared_inter
        h = _vp()
        d = OfficialDesc(hidden, shared_inter, router_experts)
        check(self.lib.k3x_hip_official_create(ctx.handle, experts.handle if experts else None,
                                               C.byref(d), C.byref(h)),
              "k3x_hip_official_create")
        self.handle = h
        if not hasattr(ctx, "_officials"):
            ctx._officials = weakref.WeakSet()
        ctx._officials.add(self)

    def upload_ffn(self, routed_down, routed_norm, routed_up, shared_gate=None, shared_up=None,
                   shared_down=None) -> int:
        import numpy as np
        arrs = [None if a is None else np.ascontiguousarray(a, dtype=np.uint16)
                for a in (routed_down, routed_norm, routed_up, shared_gate, shared_up,
                          shared_down)]
        return self.lib.k3x_hip_official_upload_ffn(self.handle, *[host_ptr(a) for a in arrs])

    def upload_route(self, residual_norm, residual_proj, post_norm, router, correction) -> int:
        import numpy as np
        arrs = [np.ascontiguousarray(a, dtype=np.uint16) for a in
                (residual_norm, residual_proj, post_norm, router)]
        corr = np.ascontiguousarray(correction, dtype=np.float32)
        return self.lib.k3x_hip_official_upload_route(self.handle, *[host_ptr(a) for a in arrs],
                                                      host_ptr(corr))

    def fill_synthetic(self, seed: int, sigma=0.02, router_sigma=0.02, proj_sigma=0.05,
                       correction_sigma=0.1) -> None:
        check(self.lib.k3x_hip_official_fill_synthetic(self.handle, seed, sigma, router_sigma,
                                                       proj_sigma, correction_sigma),
              "k3x_hip_official_fill_synthetic")

    def prepare(self, tokens, eps, prefix, residual, hidden, logits=None) -> int:
        return self.lib.k3x_hip_official_prepare(self.ctx.handle, self.handle, tokens, eps,
                                                 ptr(prefix), ptr(residual), ptr(hidden),
                                                 ptr(logits))

    def ffn(self, params: "MoeParams", hidden, prefix, out, ids=None, contributions=None,
            taps=None) -> int:
        t = None
        if taps:
            t = OfficialTaps()
            for k, v in taps.items():
                if k not in OFFICIAL_TAP_FIELDS:
                    raise ValueError(f"unknown tap {k!r}; taps are {OFFICIAL_TAP_FIELDS}")
                setattr(t, k, ptr(v))
        return self.lib.k3x_hip_official_ffn(self.ctx.handle, self.handle, C.byref(params),
                                             ptr(hidden), ptr(prefix), ptr(ids),
                                             ptr(contributions), ptr(out),
                                             C.byref(t) if t is not None else None)

    def close(self) -> None:
        if self.handle:
            self.lib.k3x_hip_official_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def make_params(tokens, top_k, routed_scale=1.0, eps=1e-6, glu=GLU_SWIGLU, beta=4.0,
                linear=None, renorm=RENORM_FLOAT, flags=0) -> MoeParams:
    return MoeParams(tokens, top_k, routed_scale, eps, glu, beta, int(linear is not None),
                     linear or 0.0, renorm, flags)


def make_taps(tensors: dict | None) -> MoeTaps | None:
    if not tensors:
        return None
    t = MoeTaps()
    for k, v in tensors.items():
        if k not in TAP_FIELDS:  # a plain attribute would be ignored by the library
            raise ValueError(f"unknown tap {k!r}; taps are {TAP_FIELDS}")
        setattr(t, k, ptr(v))
    return t


def synth_normal_bf16(ctx: Context, seed: int, stream: int, sigma: float, out) -> None:
    check(ctx.lib.k3x_hip_synth_normal_bf16(ctx.handle, seed, stream, sigma, out.numel(),
                                            ptr(out)), "k3x_hip_synth_normal_bf16")


def moe_forward(ctx: Context, bank: Bank, params: MoeParams, x, out, taps=None) -> int:
    t = make_taps(taps)
    return ctx.lib.k3x_hip_moe_forward(ctx.handle, bank.handle, C.byref(params), ptr(x),
                                       ptr(out), C.byref(t) if t is not None else None)


def moe_forward_noalloc(ctx: Context, bank: Bank, params: MoeParams, x, out, taps=None) -> int:
    """k3x_hip_moe_forward over the library's fixed device scratch (no device
    allocation in the call)."""
    t = make_taps(taps)
    return ctx.lib.k3x_hip_moe_forward_noalloc(ctx.handle, bank.handle, C.byref(params), ptr(x),
                                               ptr(out), C.byref(t) if t is not None else None)


def moe_forward_routed(ctx: Context, bank: Bank, params: MoeParams, xn, ids, weights, out,
                       host_ids=None, host_weights=None, taps=None) -> int:
    t = make_taps(taps)
    return ctx.lib.k3x_hip_moe_forward_routed(
        ctx.handle, bank.handle, C.byref(params), ptr(xn), ptr(ids), ptr(weights),
        host_ptr(host_ids), host_ptr(host_weights), ptr(out),
        C.byref(t) if t is not None else None)


def dense_f32_matvec(ctx: Context, W, x, y) -> int:
    """y [T][rows] = W [rows][cols] x [T][cols] (fp32 device tensors)."""
    rows, cols = W.shape
    T = x.numel() // cols
    return load().k3x_hip_dense_f32_matvec(ctx.handle, ptr(W), rows, cols, ptr(x), T, ptr(y))


def mxfp4_matvec(ctx: Context, packed, scales, rows: int, cols: int, x, y) -> int:
    """y [T][rows] = an MXFP4 matrix (K3X layout, device uint8 tensors) x."""
    T = x.numel() // cols
    return load().k3x_hip_mxfp4_matvec(ctx.handle, ptr(packed), ptr(scales), rows, cols, ptr(x),
                                       T, ptr(y))


def dense_situ_mlp(ctx: Context, gate, up, down, x, act, y, beta=4.0, linear=None) -> int:
    inter, hidden = gate.shape
    out_rows = down.shape[0]
    T = x.numel() // hidden
    return load().k3x_hip_dense_situ_mlp(ctx.handle, ptr(gate), ptr(up), ptr(down), hidden,
                                         inter, out_rows, beta, int(linear is not None),
                                         linear or 0.0, ptr(x), T, ptr(act), ptr(y))


def resident_moe_layer(ctx: Context, bank: "Bank", weights: dict, params: MoeParams, x, ids,
                       contributions, out, mixed=None, host_ids=None,
                       host_contributions=None) -> int:
    """The resident latent layer: weights is a dict of fp32 device tensors
    (routed_down [L][H], routed_norm [L], routed_up [H][L], shared_gate /
    shared_up [S][H], shared_down [H][S])."""
    L, H = weights["routed_down"].shape
    S = weights["shared_gate"].shape[0]
    w = LatentWeights(*[ptr(weights[k]) for k in ("routed_down", "routed_norm", "routed_up",
                                                  "shared_gate", "shared_up", "shared_down")],
                      H, L, S, 0)
    return load().k3x_hip_resident_moe_layer(
        ctx.handle, bank.handle, C.byref(w), C.byref(params), ptr(x), ptr(ids),
        ptr(contributions), host_ptr(host_ids), host_ptr(host_contributions), ptr(out),
        ptr(mixed))


def expert_major_plan(ctx: Context, ids, tokens, top_k, experts, taps: dict) -> int:
    t = make_taps(taps)
    return ctx.lib.k3x_hip_expert_major_plan(ctx.handle, ptr(ids), tokens, top_k, experts,
                                             C.byref(t))


class Storage:
    """A K3X checkpoint opened for expert loads (k3x_hip_storage_*).  Opening
    is host work only; status() is the open's status code."""

    def __init__(self, path: str):
        self.lib = load()
        h = _vp()
        self.open_status = self.lib.k3x_hip_storage_open(path.encode(), C.byref(h))
        self.handle = h if self.open_status == 0 else None

    def upload_expert(self, bank: "Bank", slot: int, layer_id: int, expert_id: int):
        """(status, bytes read) of load_storage_expert into bank slot `slot`."""
        n = C.c_uint64(0)
        st = self.lib.k3x_hip_storage_upload_expert(self.handle, bank.handle, slot, layer_id,
                                                    expert_id, C.byref(n), None)
        return st, n.value

    def upload_expert_digest(self, bank: "Bank", slot: int, layer_id: int, expert_id: int):
        """(status, bytes read, the six extents' ordered SHA-256 as 32 bytes)."""
        n = C.c_uint64(0)
        d = (C.c_uint8 * 32)()
        st = self.lib.k3x_hip_storage_upload_expert(self.handle, bank.handle, slot, layer_id,
                                                    expert_id, C.byref(n), C.cast(d, C.c_void_p))
        return st, n.value, bytes(d)

    def verify(self) -> int:
        """Reader::open's checksums verification: tensor CRC32Cs, directory and
        root SHA-256 (status code)."""
        return self.lib.k3x_hip_storage_verify(self.handle)

    def close(self) -> None:
        if self.handle:
            self.lib.k3x_hip_storage_close(self.handle)
            self.handle = None
