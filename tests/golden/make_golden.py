#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ from the reference's own CPU
functions (oracle/_ref/libk3x_ref.so, compiled in place from the reference
sources by `make -C oracle ref`).  Run in the container that holds the
reference tree; the GPU box only reads the .npz files.

Inputs come from the build's seeded generator (tests/synth.py), so every
fixture is regenerated bit-identically from its seed.

  c1_layer.npz   config-1 layer (H=256, E=16, I=512, Top-4), 8 tokens,
                 the reference composition per token (rms_norm -> router ->
                 sigmoid -> select_routing -> mxfp4_situ_moe): Top-4 ids and
                 fp32 outputs with SiTU beta=4 and beta=4/linear=25.
  routes_c3.npz  Top-16 ids and weights of configs 3, 4 (Zipf bias) and 5
  routes_c4.npz  (T = 2, 64, 2048) through the reference's rms_norm,
  routes_c5.npz  dense_matvec and select_routing at the layer's rounding
                 point (normalised input rounded to bf16 before the router).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

from oracle import Oracle, RefLib, bf16_to_f32  # noqa: E402
from synth import CONFIGS, SynthLayer, sid, STREAM_INPUT  # noqa: E402


def c1_layer(o: Oracle, ref: RefLib) -> None:
    cfg = CONFIGS[1]
    layer = SynthLayer(o, cfg)
    T = 8
    x_bits = o.synth_normal_bf16(o.stream_key(cfg.x_seed, sid(STREAM_INPUT)), T * cfg.hidden,
                                 1.0).reshape(T, cfg.hidden)
    x = bf16_to_f32(x_bits)
    experts = [layer.expert(e) for e in range(cfg.experts)]
    out = {}
    for name, linear in (("situ", None), ("situ_linear", 25.0)):
        ids = np.zeros((T, cfg.top_k), np.uint32)
        y = np.zeros((T, cfg.hidden), np.float32)
        for t in range(T):
            st, ids[t], y[t] = ref.moe_layer_token(x[t], layer.gamma, cfg.eps, layer.router,
                                                   layer.bias, experts, cfg.hidden, cfg.inter,
                                                   cfg.top_k, cfg.routed_scale, None, beta=4.0,
                                                   linear=linear)
            assert st == 0, st
        out["ids"] = ids
        out[f"out_{name}"] = y
    np.savez_compressed(os.path.join(HERE, "c1_layer.npz"), x_bits=x_bits, seed=cfg.seed,
                        x_seed=cfg.x_seed, **out)


def routes(o: Oracle, ref: RefLib, cid: int) -> None:
    cfg = CONFIGS[cid]
    layer = SynthLayer(o, cfg)
    x = bf16_to_f32(layer.x_bits())
    st, ids, w = ref.route_tokens(x, layer.gamma, cfg.eps, layer.router, layer.bias, cfg.top_k,
                                  cfg.routed_scale, round_normed=True)
    assert st == 0, st
    np.savez_compressed(os.path.join(HERE, f"routes_c{cid}.npz"), ids=ids.astype(np.uint16),
                        weights=w, seed=cfg.seed, x_seed=cfg.x_seed, tokens=cfg.tokens)
    print(f"config {cid}: {ids.shape[0]} tokens routed")


def main() -> None:
    o, ref = Oracle(), RefLib()
    c1_layer(o, ref)
    for cid in (3, 4, 5):
        routes(o, ref, cid)


if __name__ == "__main__":
    main()
