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


def test_upload_replaces_slot_identity(hip):
    """A slot uploaded again holds the new expert only: the old tensor ids stop
    resolving to it and may be admitted into another slot (exact residency,
    runtime/cuda/resident_weights.cu:107-166)."""
    k3x_amd, ctx = hip
    bank = k3x_amd.Bank(ctx, k3x_amd.LayerShape(hidden=128, inter=128, experts=2))
    n = 128 * 128
    ex = dict(gate_packed=np.zeros(n // 2, np.uint8), gate_scales=np.full(n // 32, 127, np.uint8),
              up_packed=np.zeros(n // 2, np.uint8), up_scales=np.full(n // 32, 127, np.uint8),
              down_packed=np.zeros(n // 2, np.uint8), down_scales=np.full(n // 32, 127, np.uint8))
    assert bank.upload_expert(0, ex, tensor_ids=(11, 12, 13)) == 0
    assert bank.upload_expert(0, ex, tensor_ids=(21, 22, 23)) == 0
    for tid in (11, 12, 13):
        assert bank.find(tid)[0] == k3x_amd.ERR_TENSOR_NOT_FOUND
    assert bank.find(22) == (0, 0, 1)
    assert bank.upload_expert(1, ex, tensor_ids=(11, 12, 13)) == 0
    assert bank.find(13) == (0, 1, 2)
    # Arguments are checked before the slot is touched: a rejected upload
    # leaves its expert resident.
    ex["gate_scales"][0] = 0xFF
    assert bank.upload_expert(1, ex, tensor_ids=(31, 32, 33)) == k3x_amd.ERR_INVALID_MXFP4
    assert bank.find(11) == (0, 1, 0)
    bank.close()


# ---------------------------------------------------------------------------
# Full layer on the seeded benchmark configurations.
# ---------------------------------------------------------------------------
def run_layer(k3x_amd, ctx, cfg, bank, x_bits, flags=0, per_pair=True, glu=None, linear=None,
              group=True):
    """One forward call with taps.  per_pair=False skips the [T][K][H] expert
    output tap (939 MB at T=2048); group=False the per-expert grouping taps
    (counts, offsets, first uses, active first uses)."""
    dev = "cuda:0"
    T, H, I, E, K = cfg.tokens, cfg.hidden, cfg.inter, cfg.experts, cfg.top_k
    x = torch.from_numpy(np.ascontiguousarray(x_bits).view(np.int16)).to(dev)
    out = torch.empty((T, H), dtype=torch.int16, device=dev)
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device=dev)
    taps = dict(normed_x=z((T, H), torch.int16), logits=z((T, E), torch.float32),
                ids=z((T, K), torch.int32), weights=z((T, K), torch.float32),
                counts=z((E,), torch.int32), offsets=z((E + 1,), torch.int32),
                pair_token=z((T * K,), torch.int32), pair_slot=z((T * K,), torch.int32),
                first_use=z((E,), torch.int32), n_active=z((1,), torch.int32),
                active_first_use=z((E,), torch.int32), act=z((T * K, I), torch.int16),
                out_f32=z((T, H), torch.float32))
    if per_pair:
        taps["expert_out"] = z((T, K, H), torch.float32)
    if not group:
        for k in ("counts", "offsets", "first_use", "active_first_use"):
            del taps[k]
    if cfg.shared_inter:
        taps["shared_out"] = z((T, H), torch.float32)
        taps["shared_act"] = z((T, cfg.shared_inter), torch.int16)
    params = k3x_amd.make_params(T, K, cfg.routed_scale, cfg.eps,
                                 cfg.glu if glu is None else glu, cfg.beta,
                                 cfg.linear if linear is None else linear, cfg.renorm, flags)
    st = k3x_amd.moe_forward(ctx, bank, params, x, out, taps)
    assert st == 0, st
    assert ctx.synchronize() == 0
    got = {k: to_np(v) for k, v in taps.items()}
    got["out"] = to_np(out)
    for k in ("ids", "counts", "offsets", "pair_token", "pair_slot", "first_use", "n_active",
              "active_first_use"):
        if k in got:
            got[k] = got[k].view(np.uint32)
    for k in ("normed_x", "act", "out", "shared_act"):
        if k in got:
            got[k] = got[k].view(np.uint16)
    return got


def check_routing(oracle, layer, got, x_bits):
    """RMSNorm, logits, Top-K ids and weights, grouping: all bit-exact."""
    cfg = layer.cfg
    T, K, E = x_bits.shape[0], cfg.top_k, cfg.experts
    xn = layer.normed(x_bits)
    xn_bits = (xn.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(got["normed_x"], xn_bits), "RMSNorm output differs"
    logits, ids, w = layer.route(xn)
    assert np.array_equal(got["logits"].view(np.uint32), logits.view(np.uint32)), "logits differ"
    assert np.array_equal(got["ids"], ids), "Top-K ids differ"
    assert np.array_equal(got["weights"].view(np.uint32), w.view(np.uint32)), "weights differ"
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
    say(f"rmsnorm, logits, ids, weights, grouping bit-exact ({na} active experts)")
    return xn, ids, w, csr


def check_threads() -> int:
    """Host threads for the checker's per-expert work (the box's CPU share)."""
    import os
    return max(1, min(16, os.cpu_count() or 1))


def check_layer(oracle, layer, got, x_bits=None, tokens_checked=None, report=None):
    """Layer outputs against the oracle (see the module docstring); `report`,
    when given, receives the figures the checks rest on.  The checked pairs
    are grouped by expert and each expert's oracle work (its pairs' double
    GEMVs, its decoded down projection and the bound products over all its
    pairs at once) runs on a pool of host threads, so that every token of a
    verification window, or hundreds of a prefill chunk, can be checked."""
    from collections import defaultdict
    from concurrent.futures import ThreadPoolExecutor
    cfg = layer.cfg
    x_bits = layer.x_bits() if x_bits is None else x_bits
    T, K, H, I = x_bits.shape[0], cfg.top_k, cfg.hidden, cfg.inter
    P = T * K
    xn, ids, w, csr = check_routing(oracle, layer, got, x_bits)
    tokens = list(range(T)) if tokens_checked is None else sorted(set(tokens_checked))
    act_gpu = got["act"]  # CSR rows
    row_of = {(int(csr["pair_token"][r]), int(csr["pair_slot"][r])): r for r in range(P)}
    by_expert = defaultdict(list)
    for t in tokens:
        for s_ in range(K):
            by_expert[int(ids[t, s_])].append((t, s_))
    threads = check_threads()
    layer.prefetch(by_expert.keys(), threads)

    def expert_work(e):
        """Activations of expert e's checked pairs against the oracle's, its
        down projection on the GPU's activations (when the per-pair outputs
        were tapped), and the propagated-bound terms |W| |da| and |W| |a|."""
        ex = layer.expert(e)
        pairs = by_expert[e]
        refs, a_cols, da_cols, stats = [], [], [], [0, 0]
        for (t, s_) in pairs:
            st, act_ref, y_ref = oracle.expert_ffn(xn[t], ex, H, I, cfg.glu, cfg.beta,
                                                   cfg.linear, round_act=True)
            assert st == 0, st
            r = row_of[(t, s_)]
            # Activations: the bf16 roundings of the GPU's fp32 sums and the
            # oracle's double sums agree except near rounding boundaries (one
            # ulp apart) and on values near zero, where the absolute
            # accumulation error of gate/up (~2^-18 of the row's scale) spans
            # more than one ulp; a layout or indexing error would be O(1) of
            # the row's scale.
            ref_bits = (act_ref.view(np.uint32) >> 16).astype(np.uint16)
            d = ulp_diff_bf16(act_gpu[r], ref_bits)
            stats[0] = max(stats[0], int(d.max()))
            frac = np.count_nonzero(d) / d.size
            assert frac < 0.02, f"pair ({t},{s_}): {frac:.4f} of activations off"
            big = d > 1
            stats[1] += int(big.sum())
            if big.any():
                scale = float(np.abs(act_ref).max())
                diff = np.abs(bf16_to_f32(act_gpu[r]) - act_ref)[big]
                assert (np.abs(act_ref[big]) <= 2.0 ** -6 * scale).all()
                assert (diff <= 2.0 ** -12 * scale).all()
            a = bf16_to_f32(act_gpu[r]).astype(np.float64)
            a_cols.append(a)
            da_cols.append(np.abs(a - act_ref.astype(np.float64)))
            refs.append(y_ref)
        st, W = oracle.decode_mxfp4(ex["down_packed"], ex["down_scales"], H, I, 32)
        assert st == 0
        W64 = W.astype(np.float64)
        Wa = np.abs(W64)
        A = np.stack(a_cols, axis=1)
        P_da = Wa @ np.stack(da_cols, axis=1)
        P_a = Wa @ np.abs(A)
        if "expert_out" in got:
            # Down projection on the GPU's own activations (isolates the
            # GEMM): fp32 accumulation over K terms is within K 2^-24 sum|w a|
            # in the worst case; 2^-16 (K = 2048 -> 2^-13 worst, ~2^-18.5
            # typical) flags any indexing or layout error, which is O(1).
            Y = W64 @ A
            for j, (t, s_) in enumerate(pairs):
                err = np.abs(got["expert_out"][t, s_].astype(np.float64) - Y[:, j])
                excess = err - 2.0 ** -16 * P_a[:, j]
                assert (excess <= 1e-30).all(), f"pair ({t},{s_}): max excess {excess.max()}"
        return {pair: (refs[j], P_da[:, j], P_a[:, j]) for j, pair in enumerate(pairs)}, stats

    with ThreadPoolExecutor(threads) as pool:
        done = list(pool.map(expert_work, sorted(by_expert)))
    per_pair, worst_act, multi = {}, 0, 0
    for res, stats in done:
        per_pair.update(res)
        worst_act = max(worst_act, stats[0])
        multi += stats[1]
    say(f"activations of {len(per_pair)} pairs over {len(by_expert)} experts: max {worst_act} "
        f"bf16 ulp, {multi} elements over 1 ulp (all near zero)")
    if "expert_out" in got:
        say("down projection within the fp32 accumulation bound on GPU activations")

    # The shared expert of every checked token: the oracle's output and
    # activation, and the bound terms of the activation differences.
    Wd = None
    if cfg.shared_inter:
        sg, su, sd = layer.shared
        Wd = np.abs(bf16_to_f32(sd)).astype(np.float64)

    def shared_work(t):
        if not cfg.shared_inter:
            return np.zeros(H, np.float32), np.zeros(H), np.zeros(H)
        sh = layer.shared_out(xn, [t])[t]
        sa_ref = round_bf16_np(oracle, xn[t], sg, su, cfg)
        sa_gpu = bf16_to_f32(got["shared_act"][t]).astype(np.float64)
        # One bf16 ulp, or near zero (as the routed activations above).
        close_acts(got["shared_act"][t][None], bf16_bits(sa_ref.astype(np.float32))[None])
        sb = Wd @ np.abs(sa_gpu - sa_ref) + 2.0 ** -15 * (Wd @ np.abs(sa_gpu))
        np.testing.assert_array_less(np.abs(got["shared_out"][t] - sh) - sb,
                                     1e-30 + 4 * 2.0 ** -24 * np.abs(sh))
        return sh, sb, np.abs(sh.astype(np.float64))

    with ThreadPoolExecutor(threads) as pool:
        shared = dict(zip(tokens, pool.map(shared_work, tokens)))

    # Against the fully independent CPU layer, element by element, with a
    # bound that accounts for every source of difference: the activation
    # elements whose bf16 rounding differs (GPU fp32 MFMA sums vs the
    # oracle's double sums land on either side of a bf16 rounding boundary;
    # each such element is one bf16 ulp apart, checked above), propagated
    # through |W_down|; fp32 accumulation of the down projections (2^-15 of
    # sum |w_rk a_k|; K = 2048 gives at most 2^-13, typically ~2^-18.5); and
    # the float rounding of the slot-ordered combine on both sides.
    within = total = 0
    u = 2.0 ** -24
    for t in tokens:
        y_t = np.stack([per_pair[(t, s_)][0] for s_ in range(K)])
        sh, sb, smag = shared[t]
        out_ref = oracle.ordered_mix(y_t, w[t]) + sh
        bound = sb.copy()
        mag = smag.copy()
        for s_ in range(K):
            y_ref, p_da, p_a = per_pair[(t, s_)]
            ws = abs(float(w[t, s_]))
            bound += ws * (p_da + 2.0 ** -15 * p_a)
            mag += ws * np.abs(y_ref.astype(np.float64))
        bound += 2 * (K + 1) * u * mag + 2 * u * np.abs(out_ref)
        err = np.abs(got["out_f32"][t].astype(np.float64) - out_ref)
        assert (err <= bound).all(), f"token {t}: {int((err > bound).sum())} outputs beyond the bound"
        ok = np.abs(got["out_f32"][t] - out_ref) <= ATOL + RTOL * np.abs(out_ref)
        within += int(ok.sum())
        total += ok.size
        assert np.array_equal(got["out"][t], bf16_bits(got["out_f32"][t]))
    frac = within / total
    say(f"{len(tokens)} tokens within the propagated bound; {frac:.5f} of outputs within "
        f"rtol {RTOL} / atol {ATOL}")
    if report:
        report(f"{len(tokens)} tokens checked: all outputs within the propagated bound; "
               f"{within}/{total} = {frac:.5f} within rtol {RTOL} / atol {ATOL}; activations "
               f"max {worst_act} bf16 ulp, {multi} elements over 1 ulp (near zero)")
    assert frac >= 0.99
    if "expert_out" in got:
        # Combine on the GPU's own per-pair outputs: bit-exact.
        sh = got["shared_out"] if cfg.shared_inter else np.zeros_like(got["out_f32"])
        comb = layer.combine(got["expert_out"], w, sh)
        assert np.array_equal(comb.view(np.uint32), got["out_f32"].view(np.uint32))
        say("ordered combine bit-exact")


def round_bf16_np(oracle, xn, gate, up, cfg):
    """The oracle's shared-expert activation bf16(GLU(gate xn, up xn))."""
    from oracle import round_bf16
    g = oracle.bf16_matvec(xn, gate)
    u = oracle.bf16_matvec(xn, up)
    a = oracle.glu(g, u, cfg.glu, cfg.beta, cfg.linear)
    return round_bf16(a).astype(np.float64)


def make_bank(k3x_amd, ctx, cfg, layer=None):
    shape = k3x_amd.LayerShape(cfg.hidden, cfg.inter, cfg.experts, cfg.shared_inter)
    bank = k3x_amd.Bank(ctx, shape)
    bank.fill_synthetic(cfg.seed, cfg.scale_lo, cfg.scale_hi, cfg.router_sigma, cfg.bias_sigma,
                        cfg.shared_sigma, 1.0)
    if cfg.zipf_b0 > 0:
        assert bank.upload_router(layer.router, layer.bias, layer.gamma) == 0
    return bank


# Router on the fp64 matrix cores (T >= 256, H <= 8192) and its fallback:
# ragged expert and token tiles (among them 8 and 16 expert tiles, the
# latter ragged), hidden sizes with padded terms, and every path that
# writes the router weights (synthetic fill, host upload, device copy)
# refreshes the residue-major copy the matrix-core router reads.
@pytest.mark.parametrize("T,H,E", [(256, 1152, 20), (300, 7168, 40), (272, 8192, 16),
                                   (257, 128, 33), (260, 8320, 18), (300, 7168, 128),
                                   (257, 1152, 250)],
                         ids=["h1152", "h7168", "h8192", "h128", "h8320_fallback",
                              "h7168_e128", "h1152_e250"])
def test_router_shapes(hip, oracle, T, H, E):
    from synth import Config, SynthLayer
    k3x_amd, ctx = hip
    cfg = Config(f"router_{T}_{H}_{E}", T, H, 128, E, 4, 0, 119, 123, routed_scale=2.5)
    say(f"router shape T={T} H={H} E={E}")
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg)
    x = layer.x_bits()
    check_routing(oracle, layer, run_layer(k3x_amd, ctx, cfg, bank, x, per_pair=False), x)
    rng = np.random.default_rng(T + H + E)
    layer.router = (rng.standard_normal((E, H)) * 0.03).astype(np.float32)
    assert bank.upload_router(layer.router, layer.bias, layer.gamma) == 0
    check_routing(oracle, layer, run_layer(k3x_amd, ctx, cfg, bank, x, per_pair=False), x)
    layer.router = (rng.standard_normal((E, H)) * 0.01).astype(np.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda:0")
    w, b, g = dev(layer.router), dev(layer.bias), dev(layer.gamma)
    assert bank.set_router_device(w, b, g) == 0
    check_routing(oracle, layer, run_layer(k3x_amd, ctx, cfg, bank, x, per_pair=False), x)
    bank.close()


# Few tokens on the general path: the register router (one, two and four
# token rows; the loop kernel past 8192 hidden) and the register Top-K (8 and
# 16 keys per lane; the LDS kernel past 1024 experts), all bit-exact.
@pytest.mark.parametrize("T,H,E", [(1, 1152, 1000), (2, 7168, 600), (3, 8192, 300),
                                   (4, 7168, 1030), (2, 8320, 700)],
                         ids=["t1", "t2", "t3", "t4_e1030", "t2_h8320"])
def test_router_few_tokens(hip, oracle, T, H, E):
    from synth import Config, SynthLayer
    k3x_amd, ctx = hip
    cfg = Config(f"route_{T}_{H}_{E}", T, H, 128, E, 8, 0, 119, 123, routed_scale=2.5)
    say(f"few-token route T={T} H={H} E={E}")
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg)
    x = layer.x_bits()
    got = run_layer(k3x_amd, ctx, cfg, bank, x, k3x_amd.FLAG_GENERAL_PATH, per_pair=False)
    check_routing(oracle, layer, got, x)
    bank.close()


@pytest.fixture(scope="module")
def c3(hip, oracle):
    from synth import CONFIGS, SynthLayer
    k3x_amd, ctx = hip
    cfg = CONFIGS[3]
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg)
    yield cfg, layer, bank
    bank.close()


@pytest.mark.parametrize("cid", [1, 2, 3])
@pytest.mark.parametrize("general", [False, True], ids=["decode_path", "general_path"])
def test_layer_parity(hip, oracle, cid, general, c3, parity_report):
    """Configs 1 (tiny layer), 2 (one K3-shaped expert, T=1, Top-1 of one
    expert, no shared expert) and 3 (the T=2 decode layer) on both paths."""
    from synth import CONFIGS, SynthLayer
    k3x_amd, ctx = hip
    cfg = CONFIGS[cid]
    say(f"layer parity config {cid} ({cfg.name}) T={cfg.tokens} general={general}")
    if cid == 3:
        _, layer, bank = c3
    else:
        layer = SynthLayer(oracle, cfg)
        bank = make_bank(k3x_amd, ctx, cfg)
    # Synthetic fill is bit-identical to the CPU generator (sampled rows).
    for e in (0, cfg.experts - 1):
        ex = layer.expert(e)
        st, want = oracle.decode_mxfp4(ex["down_packed"][: 4 * cfg.inter // 2],
                                       ex["down_scales"][: 4 * cfg.inter // 32], 4, cfg.inter)
        got = to_np(bank.dequant_rows(e, 2, 0, 4))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    flags = k3x_amd.FLAG_GENERAL_PATH if general else 0
    got = run_layer(k3x_amd, ctx, cfg, bank, layer.x_bits(), flags)
    check_layer(oracle, layer, got, report=parity_report)
    if cid != 3:
        bank.close()


def close_paths(a, b):
    """Two fp32 results that differ in fp32 summation orders and, through
    those, in a few bf16 activation roundings on each side: within 2^-10 of
    each other in norm and element-wise within the layer tolerance on >= 97%
    of elements (the misses are small outputs where a flipped activation
    rounding is a large relative change; each path is checked element by
    element against the oracle with a propagated bound in check_layer)."""
    ok = np.abs(a - b) <= ATOL + RTOL * np.abs(b)
    assert ok.mean() >= 0.97
    assert np.linalg.norm(a - b) <= 2.0 ** -10 * np.linalg.norm(b)


def close_acts(a, b):
    """bf16 activations of two paths whose fp32 sums differ in order: equal
    or one ulp apart except on values near zero (see check_layer)."""
    d = ulp_diff_bf16(a, b)
    assert np.count_nonzero(d) / d.size < 0.02
    big = d > 1
    if big.any():
        fa, fb = bf16_to_f32(a).astype(np.float64), bf16_to_f32(b).astype(np.float64)
        scale = np.abs(fb).max(axis=-1, keepdims=True) * np.ones_like(fb)
        assert (np.abs(fb[big]) <= 2.0 ** -6 * scale[big]).all()
        assert (np.abs(fa - fb)[big] <= 2.0 ** -12 * scale[big]).all()


def test_decode_and_general_paths_agree(hip, c3):
    """Both paths: normalisation, routing and grouping bit-identical; the
    activations, per-pair outputs, shared expert and output agree to the
    rounding of their different fp32 summation orders (the decode path splits
    K ranges over waves)."""
    k3x_amd, ctx = hip
    cfg, layer, bank = c3
    x = layer.x_bits()
    a = run_layer(k3x_amd, ctx, cfg, bank, x, 0)
    b = run_layer(k3x_amd, ctx, cfg, bank, x, k3x_amd.FLAG_GENERAL_PATH)
    for k in ("normed_x", "logits", "ids", "weights", "counts", "offsets", "first_use",
              "n_active", "active_first_use", "pair_token", "pair_slot"):
        assert np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), k
    close_acts(a["act"], b["act"])
    close_acts(a["shared_act"], b["shared_act"])
    close_paths(a["expert_out"], b["expert_out"])
    close_paths(a["shared_out"], b["shared_out"])
    close_paths(a["out_f32"], b["out_f32"])


def test_repeated_decode_calls(hip, oracle, c3):
    """Back-to-back decode calls with different inputs, including T=1 calls
    (per-call buffers of one call must not leak into the next): each call's
    routing and grouping bit-exact, its output equal to the general path's."""
    from synth import sid, STREAM_INPUT
    k3x_amd, ctx = hip
    cfg, layer, bank = c3
    import dataclasses
    # Every decode-path token count, 1 to 4 (16 to 64 pairs).
    for i, T in enumerate((2, 2, 1, 2, 1, 4, 3)):
        x = oracle.synth_normal_bf16(oracle.stream_key(cfg.x_seed + 100 + i, sid(STREAM_INPUT)),
                                     T * cfg.hidden, 1.0).reshape(T, cfg.hidden)
        c = dataclasses.replace(cfg, tokens=T)
        a = run_layer(k3x_amd, ctx, c, bank, x, 0, per_pair=False)
        b = run_layer(k3x_amd, ctx, c, bank, x, k3x_amd.FLAG_GENERAL_PATH, per_pair=False)
        check_routing(oracle, layer, a, x)
        close_acts(a["act"][: T * cfg.top_k], b["act"][: T * cfg.top_k])
        close_paths(a["out_f32"], b["out_f32"])
        say(f"call {i} (T={T}) ok")


def test_decode_deterministic(hip, c3):
    k3x_amd, ctx = hip
    cfg, layer, bank = c3
    x = layer.x_bits()
    a = run_layer(k3x_amd, ctx, cfg, bank, x, 0, per_pair=False)
    b = run_layer(k3x_amd, ctx, cfg, bank, x, 0, per_pair=False)
    for k in a:
        assert np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), k


@pytest.mark.parametrize("cid,T,E", [(1, 1, None), (1, 2, None), (1, 4, None), (2, 1, None),
                                     (2, 3, None), (1, 2, 4), (1, 3, 3)])
def test_small_route_two_launches(hip, oracle, cid, T, E):
    """Few experts, no shared expert (configs 1 and 2): without the
    per-expert grouping taps the decode path runs in two launches, every
    gate/up workgroup finding the route itself.  Everything it writes equals
    the four-launch form's (taken with those taps, whose routing is checked
    against the oracle here) bit for bit: the same xn, logits, Top-K,
    grouping, activations, per-pair rows and output.  E <= K (config 2, and
    config 1 cut to 4 or 3 experts with Top-4 / Top-3) takes the form where
    every expert is active and its weights are requested before the route
    is known."""
    import dataclasses
    from synth import CONFIGS, SynthLayer
    k3x_amd, ctx = hip
    cfg = dataclasses.replace(CONFIGS[cid], tokens=T)
    if E is not None:
        cfg = dataclasses.replace(cfg, experts=E, top_k=E)
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg)
    x = layer.x_bits()
    say(f"two-launch decode config {cid} T={T}")
    launches = lambda: ctx.stats().kernel_launches
    n0 = launches()
    a = run_layer(k3x_amd, ctx, cfg, bank, x, 0, group=False)
    n1 = launches()
    b = run_layer(k3x_amd, ctx, cfg, bank, x, 0, group=True)
    n2 = launches()
    assert (n1 - n0, n2 - n1) == (2, 4), (n1 - n0, n2 - n1)
    check_routing(oracle, layer, b, x)
    for k in ("normed_x", "logits", "ids", "weights", "pair_token", "pair_slot", "n_active",
              "act", "expert_out", "out_f32", "out"):
        assert np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), k
    # Back-to-back calls leave nothing behind: the same call again.
    c = run_layer(k3x_amd, ctx, cfg, bank, x, 0, group=False)
    assert np.array_equal(c["out"], a["out"])
    bank.close()


def test_c1_situ_against_reference_golden(hip, oracle):
    """Config 1 with SiTU (beta 4, linear 25): device ids equal the ids the
    reference's own CPU functions chose (tests/golden/c1_layer.npz), and the
    output is within the bf16 contract's bound of the reference output."""
    import os
    from synth import CONFIGS, SynthLayer
    from oracle import GLU_SITU
    k3x_amd, ctx = hip
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "c1_layer.npz"))
    cfg = CONFIGS[1]
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg)
    import dataclasses
    c8 = dataclasses.replace(cfg, tokens=8)
    got = run_layer(k3x_amd, ctx, c8, bank, g["x_bits"], 0, glu=GLU_SITU, linear=25.0)
    assert np.array_equal(got["ids"], g["ids"])
    for t in range(8):
        ref = g["out_situ_linear"][t]
        assert np.linalg.norm(got["out_f32"][t] - ref) <= 2.0 ** -7 * np.linalg.norm(ref)
    bank.close()


def tokens_by_row_class(got, K, classes):
    """One token per class of grouped-GEMM work item.  The grouping's CSR
    rows of expert e are [offsets[e], offsets[e+1]); a work item is a chunk of
    `chunk` consecutive rows of one expert.  classes: name -> predicate on
    (rows in the chunk, whether the chunk is its expert's last).  Returns
    {name: token} for every class some chunk falls in, taking the chunk's
    last row (so partial chunks check their final, ragged row)."""
    counts, offsets = got["counts"], got["offsets"]
    picked = {}
    for e in np.argsort(-counts.astype(np.int64), kind="stable"):
        c = int(counts[e])
        if not c:
            break
        for name, (chunk, pred) in classes.items():
            if name in picked:
                continue
            for m0 in range(0, c, chunk):
                rows = min(chunk, c - m0)
                if pred(rows, m0 + chunk >= c):
                    picked[name] = int(got["pair_token"][int(offsets[e]) + m0 + rows - 1])
                    break
    return picked


def test_wide_class_boundaries(hip, oracle):
    """The wide path's per-class launches at every class boundary: a host
    route (k3x_hip_moe_forward_routed, T = 1028, Top-2, 16 experts) gives the
    experts 32, 33, 64, 65, 96, 97, 128, 129, 160, 161, 192, 193, 224, 225,
    256 and 1 rows, so the 128-row chunks' last parts fall on both sides of
    each boundary of the classes (<= 32, 33-64, 65-96, > 96 rows) and full
    chunks come one, two and three to an expert.  Grouping bit-exact against
    the oracle's CSR; every pair's activations against the oracle's expert
    FFN; every pair's fp32 output against the down projection of the GPU's
    own activations within 2^-16 of sum |w a|; the ordered mix bit-exact on
    the GPU's per-pair rows."""
    from synth import Config, SynthLayer
    k3x_amd, ctx = hip
    counts = [32, 33, 64, 65, 96, 97, 128, 129, 160, 161, 192, 193, 224, 225, 256, 1]
    E, K = len(counts), 2
    T = sum(counts) // K
    H = I = 512
    cfg = Config("wide_classes", T, H, I, E, K, 0, 119, 123)
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg)
    # Pair list sorted by expert, split in halves: token t takes entries t and
    # t + T (distinct experts: no expert holds more than T rows).
    flat = np.repeat(np.arange(E, dtype=np.uint32), counts)
    ids = np.stack([flat[:T], flat[T:]], axis=1)
    assert (ids[:, 0] != ids[:, 1]).all()
    rng = np.random.default_rng(11)
    w = rng.uniform(0.2, 1.0, (T, K)).astype(np.float32)
    xn = layer.normed(layer.x_bits())
    xn_bits = (xn.view(np.uint32) >> 16).astype(np.uint16)
    dev = "cuda:0"
    d_xn = torch.from_numpy(xn_bits.view(np.int16)).to(dev)
    d_ids = torch.from_numpy(ids.view(np.int32)).to(dev)
    d_w = torch.from_numpy(w).to(dev)
    out = torch.empty((T, H), dtype=torch.int16, device=dev)
    z = lambda shape, dt: torch.empty(shape, dtype=dt, device=dev)
    taps = dict(counts=z((E,), torch.int32), offsets=z((E + 1,), torch.int32),
                pair_token=z((T * K,), torch.int32), pair_slot=z((T * K,), torch.int32),
                act=z((T * K, I), torch.int16), expert_out=z((T, K, H), torch.float32),
                out_f32=z((T, H), torch.float32))
    params = k3x_amd.make_params(T, K, 1.0, cfg.eps, cfg.glu, cfg.beta, cfg.linear, cfg.renorm)
    say(f"wide class boundaries: T={T} K={K} E={E} H={H} I={I}, rows per expert {counts}")
    st = k3x_amd.moe_forward_routed(ctx, bank, params, d_xn, d_ids, d_w, out, taps=taps)
    assert st == 0, st
    assert ctx.synchronize() == 0
    got = {k: to_np(v) for k, v in taps.items()}
    for k in ("counts", "offsets", "pair_token", "pair_slot"):
        got[k] = got[k].view(np.uint32)
    act = got["act"].view(np.uint16)
    st, csr = oracle.expert_major_csr(ids, E)
    assert st == 0
    assert np.array_equal(got["counts"], np.array(counts, np.uint32))
    for k in ("counts", "offsets", "pair_token", "pair_slot"):
        assert np.array_equal(got[k][:len(csr[k])], csr[k]), k
    worst_act = 0
    for e in range(E):
        ex = layer.expert(e)
        st, W = oracle.decode_mxfp4(ex["down_packed"], ex["down_scales"], H, I, 32)
        assert st == 0
        W64 = W.astype(np.float64)
        r0, r1 = int(csr["offsets"][e]), int(csr["offsets"][e + 1])
        for r in range(r0, r1):
            t, s_ = int(csr["pair_token"][r]), int(csr["pair_slot"][r])
            st, act_ref, _ = oracle.expert_ffn(xn[t], ex, H, I, cfg.glu, cfg.beta, cfg.linear,
                                               round_act=True)
            assert st == 0, st
            ref_bits = (act_ref.view(np.uint32) >> 16).astype(np.uint16)
            d = ulp_diff_bf16(act[r], ref_bits)
            worst_act = max(worst_act, int(d.max()))
            assert np.count_nonzero(d) / d.size < 0.02, f"expert {e} row {r - r0}: activations off"
            a = bf16_to_f32(act[r]).astype(np.float64)
            y = W64 @ a
            err = np.abs(got["expert_out"][t, s_].astype(np.float64) - y)
            assert (err <= 2.0 ** -16 * (np.abs(W64) @ np.abs(a)) + 1e-30).all(), \
                f"expert {e} row {r - r0} (token {t} slot {s_}): down output off"
    for t in range(T):
        mix = oracle.ordered_mix(got["expert_out"][t], w[t])
        assert np.array_equal(got["out_f32"][t].view(np.uint32), mix.view(np.uint32)), t
    say(f"wide class boundaries: grouping bit-exact, {T * K} pairs checked "
        f"(activations within {worst_act} bf16 ulp), ordered mix bit-exact")
    bank.close()


def test_c4_verification_window(hip, oracle, parity_report):
    """Config 4: T=64, Zipf-skewed routing (0..~40 rows per expert).  Routing
    and grouping bit-exact for all 1024 pairs; activations and outputs of
    every token (their pairs cover the busiest expert, mid-sized ones and
    single-row experts)."""
    from synth import CONFIGS, SynthLayer
    k3x_amd, ctx = hip
    cfg = CONFIGS[4]
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg, layer)
    got = run_layer(k3x_amd, ctx, cfg, bank, layer.x_bits())
    counts = got["counts"]
    say(f"c4 rows per expert: max {counts.max()}, active {int((counts > 0).sum())}")
    assert counts.max() >= 30
    big = lambda rows, last: rows >= 30
    picked = tokens_by_row_class(got, cfg.top_k, {
        "busiest": (1 << 30, big), "mid_8_to_29": (1 << 30, lambda r, l: 8 <= r < 30),
        "two_to_seven": (1 << 30, lambda r, l: 2 <= r < 8), "single": (1 << 30, lambda r, l: r == 1)})
    say(f"c4 row classes {picked}; checking all {cfg.tokens} tokens")
    assert len(picked) == 4
    check_layer(oracle, layer, got, tokens_checked=range(cfg.tokens), report=parity_report)
    bank.close()


# Verification windows between the decode path and the wide GEMM (4 < T <=
# 64): the routed experts run on the decode gate/up and down kernels with a
# slot's rows staged through LDS four at a time.  Cases: few rows per expert
# (T=9); Zipf-skewed slots of many rows, most not a multiple of four (T=40);
# I=3072, whose down projection holds 24 code tiles (T=64, 16 experts).
WINDOWS = {
    "t9": dict(tokens=9, hidden=1024, inter=512, experts=64, top_k=8, shared_inter=256),
    "t40_skew": dict(tokens=40, hidden=2048, inter=1024, experts=32, top_k=4, shared_inter=0,
                     zipf_b0=0.45),
    "t64_i3072": dict(tokens=64, hidden=1024, inter=3072, experts=16, top_k=4,
                      shared_inter=512),
}


@pytest.mark.parametrize("name", list(WINDOWS))
def test_verification_window_rows(hip, oracle, name, parity_report):
    from synth import Config, SynthLayer
    k3x_amd, ctx = hip
    cfg = Config(f"window_{name}", scale_lo=120, scale_hi=124, routed_scale=2.5,
                 **WINDOWS[name])
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg, layer)
    got = run_layer(k3x_amd, ctx, cfg, bank, layer.x_bits())
    counts = got["counts"]
    say(f"window {name}: T={cfg.tokens} rows per expert max {counts.max()}, "
        f"active {int((counts > 0).sum())}, slots over four rows "
        f"{int((counts > 4).sum())}, not a multiple of four {int((counts % 4 != 0).sum())}")
    if name != "t9":
        assert (counts > 4).any() and (counts[counts > 4] % 4 != 0).any()
    check_layer(oracle, layer, got, report=parity_report)
    bank.close()


def test_c5_prefill_chunk(hip, oracle, parity_report):
    """Config 5: T=2048 prefill chunk.  Device Top-16 ids equal the ids the
    reference's CPU functions chose (golden fixture); grouping bit-exact;
    outputs of every 16th token (128 tokens, 2048 pairs) plus tokens chosen
    so that a checked pair falls in each size class of the wide grouped
    GEMM's launches (128-row chunks: full and 97-127 rows at 8 row tiles,
    65-96 at 6, 33-64 at 4, at most 32 at 2; partial last chunks) and the
    last token;
    permuting the tokens permutes the output bit for bit (rows of the grouped
    GEMMs are independent)."""
    import os
    from synth import CONFIGS, SynthLayer
    k3x_amd, ctx = hip
    cfg = CONFIGS[5]
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg)
    x = layer.x_bits()
    got = run_layer(k3x_amd, ctx, cfg, bank, x, per_pair=False)
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "routes_c5.npz"))
    assert np.array_equal(got["ids"], g["ids"].astype(np.uint32))
    say("c5 ids equal the reference's")
    ch = 128
    picked = tokens_by_row_class(got, cfg.top_k, {
        "full_128": (ch, lambda r, last: r == ch),
        "partial_97_127": (ch, lambda r, last: 96 < r < ch),
        "partial_65_96": (ch, lambda r, last: 64 < r <= 96),
        "partial_33_64": (ch, lambda r, last: 32 < r <= 64 and last),
        "partial_le_32": (ch, lambda r, last: r <= 32 and last)})
    tokens = sorted(set(picked.values()) | set(range(0, cfg.tokens, 16)) | {cfg.tokens - 1})
    say(f"c5: {len(tokens)} tokens checked, item classes {picked}")
    assert len(picked) == 5 and len(tokens) >= 128
    check_layer(oracle, layer, got, x, tokens_checked=tokens, report=parity_report)
    perm = np.random.default_rng(5).permutation(cfg.tokens)
    gp = run_layer(k3x_amd, ctx, cfg, bank, x[perm], per_pair=False)
    assert np.array_equal(gp["out"], got["out"][perm])
    assert np.array_equal(gp["out_f32"].view(np.uint32), got["out_f32"][perm].view(np.uint32))
    say("c5 token permutation equivariance bit-exact")
    bank.close()


def test_c5_prefill_scaled_fp4(hip, oracle, parity_report):
    """Config 5 on the scaled FP4 MFMA (K3X_FLAG_SCALED_FP4): the routed
    experts take xn and act as two-term E4M3 rows against the MXFP4 codes as
    stored.  Routing and grouping bit-exact and permutation equivariance
    bit-exact as on the bf16 path; outputs of tokens in every work-item class
    against the oracle, with the fractions within rtol 2e-3 / atol 1e-3 and
    within 1e-2 / 5e-3 reported.  The MFMA sums each 32-element block's
    products in a window of about 2^-13 of the block's largest product (not
    in fp32), so this path does not meet the fp32-accumulation standard the
    bf16 path meets; the bounds asserted here are the measured ones."""
    from synth import CONFIGS, SynthLayer
    k3x_amd, ctx = hip
    cfg = CONFIGS[5]
    layer = SynthLayer(oracle, cfg)
    bank = make_bank(k3x_amd, ctx, cfg)
    x = layer.x_bits()
    got = run_layer(k3x_amd, ctx, cfg, bank, x, flags=k3x_amd.FLAG_SCALED_FP4, per_pair=False)
    xn, ids, w, csr = check_routing(oracle, layer, got, x)
    ch = 128
    picked = tokens_by_row_class(got, cfg.top_k, {
        "full_128": (ch, lambda r, last: r == ch),
        "partial_97_127": (ch, lambda r, last: 96 < r < ch),
        "partial_65_96": (ch, lambda r, last: 64 < r <= 96),
        "partial_33_64": (ch, lambda r, last: 32 < r <= 64 and last),
        "partial_le_32": (ch, lambda r, last: r <= 32 and last)})
    tokens = sorted(set(picked.values()) | {0, cfg.tokens - 1})
    assert len(picked) == 5
    act_ref, y_ref = layer.pair_outputs(xn, ids, tokens)
    shared = layer.shared_out(xn, tokens)
    out_ref = layer.combine(y_ref, w, shared, tokens)
    ref = np.stack([out_ref[t] for t in tokens]).astype(np.float64)
    gpu = np.stack([got["out_f32"][t] for t in tokens]).astype(np.float64)
    err = np.abs(gpu - ref)
    f_tight = float(np.mean(err <= ATOL + RTOL * np.abs(ref)))
    f_loose = float(np.mean(err <= 5e-3 + 1e-2 * np.abs(ref)))
    scale = np.abs(ref).max(axis=1, keepdims=True)
    worst = float((err / scale).max())
    # Activations against the bf16-dequant path's (same grouping, CSR rows).
    base = run_layer(k3x_amd, ctx, cfg, bank, x, per_pair=False)
    d_act = ulp_diff_bf16(got["act"], base["act"])
    msg = (f"c5 scaled FP4: {len(tokens)} tokens; {f_tight:.4f} of outputs within rtol {RTOL} / "
           f"atol {ATOL}, {f_loose:.4f} within 1e-2 / 5e-3, max |err| / row max {worst:.2e}; "
           f"activations vs bf16 path: {np.count_nonzero(d_act) / d_act.size:.4f} differ, "
           f"max {int(d_act.max())} bf16 ulp")
    say(msg)
    parity_report(msg)
    assert f_tight >= 0.9 and f_loose >= 0.99 and worst < 1e-2
    perm = np.random.default_rng(5).permutation(cfg.tokens)
    gp = run_layer(k3x_amd, ctx, cfg, bank, x[perm], flags=k3x_amd.FLAG_SCALED_FP4,
                   per_pair=False)
    assert np.array_equal(gp["out_f32"].view(np.uint32), got["out_f32"][perm].view(np.uint32))
    say("c5 scaled: token permutation equivariance bit-exact")
    bank.close()
