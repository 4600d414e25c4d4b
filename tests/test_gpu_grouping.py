"""GPU expert-major grouping (k3x_hip_expert_major_plan) against the oracle.

The device grouping takes tokens in chunks (64 tokens, or 1024 / top_k), so
the cases cover one partial chunk, several chunks with a ragged last one,
top_k = 64 (16-token chunks), 4,096 experts and skewed routes.  Bit-exact:
counts, offsets, pair_token, pair_slot, first_use, n_active and the
first-use order.  Rejections follow build_expert_major_plan
(runtime/src/expert_major.cpp:30-35): an id out of range or one expert
twice in one token latches invalid_state, reported by the next
synchronisation, after which the context works again.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

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


def routes(rng, T, K, E, skew=0.0):
    """T tokens of K distinct experts; skew > 0 favours low expert ids."""
    w = np.exp(-skew * np.arange(E) / E)
    w /= w.sum()
    ids = np.empty((T, K), np.uint32)
    for t in range(T):
        ids[t] = rng.choice(E, size=K, replace=False, p=w)
    return ids


def run_plan(k3x, ctx, ids, E):
    T, K = ids.shape
    P = T * K
    dev = torch.from_numpy(ids.astype(np.int32)).cuda()
    out = {k: torch.zeros(n, dtype=torch.int32, device="cuda:0")
           for k, n in (("counts", E), ("offsets", E + 1), ("pair_token", P), ("pair_slot", P),
                        ("first_use", E), ("n_active", 1), ("active_first_use", E))}
    st = k3x.expert_major_plan(ctx, dev, T, K, E, out)
    return st, out


CASES = [(1, 16, 384, 0.0), (5, 4, 16, 0.0), (64, 16, 384, 0.0), (200, 16, 384, 3.0),
         (2048, 16, 384, 0.0), (37, 64, 4096, 0.0), (300, 1, 7, 0.0), (129, 8, 4096, 6.0)]


@pytest.mark.parametrize("T,K,E,skew", CASES)
def test_grouping_bitexact(hip, oracle, T, K, E, skew):
    k3x, ctx = hip
    ids = routes(np.random.default_rng(T * 1000 + K * 10 + E), T, K, E, skew)
    say(f"grouping T={T} K={K} E={E} skew={skew}")
    st, out = run_plan(k3x, ctx, ids, E)
    assert st == 0
    assert ctx.synchronize() == 0
    got = {k: v.cpu().numpy().view(np.uint32) for k, v in out.items()}
    ost, csr = oracle.expert_major_csr(ids, E)
    assert ost == 0
    for k in ("counts", "offsets", "first_use"):
        assert np.array_equal(got[k], csr[k]), k
    assert np.array_equal(got["pair_token"], csr["pair_token"])
    assert np.array_equal(got["pair_slot"], csr["pair_slot"])
    na = int(got["n_active"][0])
    assert na == csr["n_active"]
    assert np.array_equal(got["active_first_use"][:na], csr["active_first_use"])


@pytest.mark.parametrize("kind", ["duplicate", "out_of_range"])
def test_grouping_rejections(hip, oracle, kind):
    k3x, ctx = hip
    T, K, E = 100, 16, 384
    ids = routes(np.random.default_rng(7), T, K, E)
    if kind == "duplicate":
        ids[70, 9] = ids[70, 2]          # second chunk, later slot repeats an earlier one
    else:
        ids[3, 15] = E
    assert oracle.expert_major_csr(ids, E)[0] == k3x.ERR_INVALID_STATE
    say(f"grouping rejects {kind}")
    st, _ = run_plan(k3x, ctx, ids, E)
    assert st == 0                       # enqueued; the kernel latches the error
    assert ctx.synchronize() == k3x.ERR_INVALID_STATE
    # The latch is cleared: a valid call on the same context succeeds.
    good = routes(np.random.default_rng(8), 10, 4, 16)
    st, out = run_plan(k3x, ctx, good, 16)
    assert st == 0 and ctx.synchronize() == 0
    ost, csr = oracle.expert_major_csr(good, 16)
    assert np.array_equal(out["pair_token"].cpu().numpy().view(np.uint32), csr["pair_token"])
