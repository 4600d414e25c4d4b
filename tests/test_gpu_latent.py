"""GPU parity of the fp32 backend operations and the resident latent MoE layer
(k3x_hip_dense_f32_matvec, k3x_hip_mxfp4_matvec, k3x_hip_dense_situ_mlp,
k3x_hip_resident_moe_layer) against the CPU oracle's restatement of
runtime/src/backend_cpu.cpp:22-122 and :305-339, which
tests/test_oracle_vs_ref.py pins bit for bit to the reference compiled in
place.

Standards:
* dense and MXFP4 matrix-vector products: every product is formed in
  double and summed in double on both sides, only the order differs, so
  every output is within one fp32 ulp of the oracle's and almost all are
  identical;
* the fp32 SiTU MLP: the device's expf / tanhf are not the host libm's
  (about one ulp each), so the activation is within 4 ulps and the output
  within 1e-5 in relative error norm;
* the resident layer: its experts run on the matrix cores (fp32 input and
  activation as bf16 hi + lo halves, fp32 accumulation) where the reference
  sums in double, so the mix and the output are within 1e-4 in relative
  error norm and every output within atol = rtol = 1e-3;
* bad arguments are rejected before any launch.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from test_oracle_vs_ref import rand_expert, rand_latent_weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

BETA, LINEAR = 4.0, 25.0


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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def to_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ulps_f32(a, b):
    ia = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, np.int64(-(2**31)) - ia, ia)
    ib = np.where(ib < 0, np.int64(-(2**31)) - ib, ib)
    return np.abs(ia - ib)


def rel_norm(got, want):
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.mark.parametrize("rows,cols,T", [(384, 7168, 1), (200, 2048, 3), (37, 101, 2),
                                         (64, 4096, 6)],
                         ids=["router", "three", "unaligned", "two_passes"])
def test_dense_f32_matvec(hip, oracle, rows, cols, T, parity_report):
    k3x_amd, ctx = hip
    say(f"dense_f32_matvec rows={rows} cols={cols} T={T}")
    rng = np.random.default_rng(rows + cols)
    W = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    y = torch.empty((T, rows), dtype=torch.float32, device="cuda:0")
    k3x_amd.check(k3x_amd.dense_f32_matvec(ctx, dev(W), dev(x), y), "dense_f32_matvec")
    got = to_np(y)
    want = np.stack([oracle.dense_matvec(x[t], W) for t in range(T)])
    u = ulps_f32(got, want)
    assert u.max() <= 1, f"max {u.max()} ulps"
    parity_report(f"{(u == 0).mean():.5f} of outputs bit-exact, the rest within 1 ulp")


def test_mxfp4_matvec(hip, oracle, parity_report):
    k3x_amd, ctx = hip
    rows, cols, T = 256, 2048, 2
    say(f"mxfp4_matvec rows={rows} cols={cols} T={T}")
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    scales = rng.integers(112, 136, rows * cols // 32, dtype=np.uint8)
    scales[:7] = [0, 1, 2, 127, 200, 251, 252]  # subnormal and large (finite) scales
    x = rng.standard_normal((T, cols)).astype(np.float32)
    x[:, :224] *= 1e-30  # keep the large-scale products finite
    y = torch.empty((T, rows), dtype=torch.float32, device="cuda:0")
    k3x_amd.check(k3x_amd.mxfp4_matvec(ctx, dev(packed), dev(scales), rows, cols, dev(x), y),
                  "mxfp4_matvec")
    got = to_np(y)
    want = np.stack([oracle.mxfp4_matvec(x[t], packed, scales, rows, cols)[1] for t in range(T)])
    u = ulps_f32(got, want)
    assert np.isfinite(want).all() and u.max() <= 1, f"max {u.max()} ulps"
    parity_report(f"{(u == 0).mean():.5f} of outputs bit-exact, the rest within 1 ulp")


@pytest.mark.parametrize("linear", [None, LINEAR], ids=["no_linear", "linear"])
def test_dense_situ_mlp(hip, oracle, linear, parity_report):
    k3x_amd, ctx = hip
    H, I, O, T = 1024, 768, 512, 2
    say(f"dense_situ_mlp H={H} I={I} O={O} T={T} linear={linear}")
    rng = np.random.default_rng(7)
    gate = (rng.standard_normal((I, H)) * 0.05).astype(np.float32)
    up = (rng.standard_normal((I, H)) * 0.05).astype(np.float32)
    down = (rng.standard_normal((O, I)) * 0.05).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    act = torch.empty((T, I), dtype=torch.float32, device="cuda:0")
    y = torch.empty((T, O), dtype=torch.float32, device="cuda:0")
    k3x_amd.check(k3x_amd.dense_situ_mlp(ctx, dev(gate), dev(up), dev(down), dev(x), act, y,
                                         BETA, linear), "dense_situ_mlp")
    got_a, got_y = to_np(act), to_np(y)
    worst_u, worst_r = 0, 0.0
    for t in range(T):
        a, want = oracle.dense_situ_mlp(x[t], gate, up, down, BETA, linear)
        worst_u = max(worst_u, int(ulps_f32(got_a[t], a).max()))
        worst_r = max(worst_r, rel_norm(got_y[t], want))
    assert worst_u <= 4 and worst_r <= 1e-5, (worst_u, worst_r)
    parity_report(f"act within {worst_u} ulps, output relative error norm {worst_r:.2e}")


def make_latent(k3x_amd, ctx, rng, H, L, I, S, E):
    w = rand_latent_weights(rng, H, L, S)
    experts = [rand_expert(rng, L, I) for _ in range(E)]
    bank = k3x_amd.Bank(ctx, k3x_amd.LayerShape(L, I, E, 0))
    for e, ex in enumerate(experts):
        k3x_amd.check(bank.upload_expert(e, ex), f"upload expert {e}")
    return w, experts, bank


@pytest.mark.parametrize("T,linear", [(1, LINEAR), (1, None), (3, LINEAR)],
                         ids=["t1", "t1_no_linear", "t3"])
def test_resident_moe_layer(hip, oracle, T, linear, parity_report):
    k3x_amd, ctx = hip
    H, L, I, S, E, K = 1024, 512, 384, 768, 12, 4
    say(f"resident_moe_layer H={H} L={L} I={I} S={S} E={E} K={K} T={T}")
    rng = np.random.default_rng(40 + T)
    w, experts, bank = make_latent(k3x_amd, ctx, rng, H, L, I, S, E)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.uint32)
    c = rng.uniform(0.1, 1.0, (T, K)).astype(np.float32)
    c /= c.sum(axis=1, keepdims=True)
    x = rng.standard_normal((T, H)).astype(np.float32)
    out = torch.empty((T, H), dtype=torch.float32, device="cuda:0")
    mixed = torch.empty((T, L), dtype=torch.float32, device="cuda:0")
    params = k3x_amd.make_params(T, K, 1.0, 1e-6, k3x_amd.GLU_SITU, BETA, linear)
    wd = {k: dev(v) for k, v in w.items()}
    st = k3x_amd.resident_moe_layer(ctx, bank, wd, params, dev(x), dev(ids.view(np.int32)),
                                    dev(c), out, mixed, host_ids=ids, host_contributions=c)
    k3x_amd.check(st, "resident_moe_layer")
    k3x_amd.check(ctx.synchronize(), "synchronize")
    got, got_m = to_np(out), to_np(mixed)
    worst, worst_m = 0.0, 0.0
    for t in range(T):
        st, want_m, want = oracle.resident_layer(x[t], w, [experts[i] for i in ids[t]], c[t],
                                                 1e-6, BETA, linear)
        assert st == 0
        worst = max(worst, rel_norm(got[t], want))
        worst_m = max(worst_m, rel_norm(got_m[t], want_m))
        np.testing.assert_allclose(got[t], want, rtol=1e-3, atol=1e-3)
    assert worst <= 1e-4 and worst_m <= 1e-4, (worst, worst_m)
    parity_report(f"mix relative error norm {worst_m:.2e}, output {worst:.2e}")
    bank.close()


def test_resident_moe_layer_rejects(hip):
    k3x_amd, ctx = hip
    H, L, I, S, E, K = 512, 256, 256, 256, 4, 2
    say("resident_moe_layer argument checks")
    rng = np.random.default_rng(9)
    w, experts, bank = make_latent(k3x_amd, ctx, rng, H, L, I, S, E)
    wd = {k: dev(v) for k, v in w.items()}
    x = dev(rng.standard_normal((1, H)).astype(np.float32))
    ids = dev(np.array([[0, 1]], np.int32))
    c = dev(np.array([[0.5, 0.5]], np.float32))
    out = torch.empty((1, H), dtype=torch.float32, device="cuda:0")
    params = k3x_amd.make_params(1, K, 1.0, 1e-6, k3x_amd.GLU_SITU, BETA, LINEAR)
    bad = k3x_amd.make_params(1, K, 1.0, 1e-6, k3x_amd.GLU_SWIGLU, BETA, LINEAR)
    assert k3x_amd.resident_moe_layer(ctx, bank, wd, bad, x, ids, c, out) == \
        k3x_amd.ERR_INVALID_MXFP4
    flagged = k3x_amd.make_params(1, K, 1.0, 1e-6, k3x_amd.GLU_SITU, BETA, LINEAR)
    flagged.flags = k3x_amd.FLAG_SPLIT_ACT
    assert k3x_amd.resident_moe_layer(ctx, bank, wd, flagged, x, ids, c, out) == \
        k3x_amd.ERR_INVALID_EXTENT
    wrong = dict(wd, routed_down=dev(w["routed_down"][:L // 2].copy()))
    assert k3x_amd.resident_moe_layer(ctx, bank, wrong, params, x, ids, c, out) == \
        k3x_amd.ERR_INVALID_EXTENT  # routed_down's rows are not the bank's latent width
    assert k3x_amd.resident_moe_layer(ctx, bank, wd, params, x, ids, c, out) == 0
    k3x_amd.check(ctx.synchronize(), "synchronize")
    bank.close()
