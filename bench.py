#!/usr/bin/env python3
"""Benchmark of the routed-expert MoE layer on one MI355X.

Workload (benchmark configuration 3 of 5, the one the headline metric is
quoted on): the K3-shaped decode layer, T=2 tokens, H=7168, 384 MXFP4
experts of I=2048, natural Top-16 with renormalised weights x2.5, one bf16
shared expert of I=2048, input RMSNorm, routing on the device.  A "step" is
one layer call.  Steps cycle over --layers resident banks (each 9 GB, a
different seed: consecutive calls stream different weights, as consecutive
layers of a decode pass do) and --inputs token pairs.

Prints one JSON line.  value = microseconds per layer call (lower is better);
the HBM figures use the bytes each call actually streams (distinct routed
experts touched x 23,396,352 B + shared expert + router).  The same line
carries the T=2048 prefill chunk as "prefill", the official K3
MoE FFN (Stable LatentMoE, at its own shapes) as "official", K3X storage
expert loads and the device CRC32C as "storage", and the reference CPU
expert path, timed on this host, as "cpu_baseline".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "project-k3x_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MXFP4_PEAK_TFLOPS = 10100.0    # MI355X dense MXFP4 / FP6
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16

H, I, E, K, S = 7168, 2048, 384, 16, 2048
EXPERT_BYTES = 3 * (H * I // 2 + H * I // 32)          # 23,396,352
GATE_UP_BYTES = 2 * (H * I // 2 + H * I // 32)         # 15,597,568
DOWN_BYTES = H * I // 2 + H * I // 32                  # 7,798,784
SHARED_GU_BYTES = 2 * S * H * 2                        # 58,720,256
SHARED_DOWN_BYTES = H * S * 2                          # 29,360,128
ROUTER_BYTES = E * H * 4 + E * 4 + H * 4               # weights + bias + gamma
EXPERT_FLOPS = 2 * 3 * H * I                           # per (token, expert) pair
SHARED_FLOPS = 2 * 3 * H * S                           # per token
SEED, X_SEED = 0x4B3358, 0x5EED
TRAFFIC_JSON_REL = "profiles/decode_c3_hbm_traffic.json"
CALIB_BYTES = 256 << 20   # plain device copy used to scale the PMC byte counters
# Bench stage -> kernel it times (for the PMC traffic of the dominant stage).
STAGE_KERNEL = {"decode_front": "decode_front_kernel", "decode_select": "decode_select_kernel",
                "decode_gate_up": "decode_gateup_kernel", "decode_down": "decode_down_kernel",
                "combine": "combine_kernel", "gate_up": "expert_gemm",
                "down": "expert_gemm"}
SCALE_LO, SCALE_HI = 119, 123


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=4, help="resident layer banks to cycle")
    ap.add_argument("--inputs", type=int, default=8, help="distinct token pairs to cycle")
    ap.add_argument("--prefill-steps", type=int, default=5)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--official-steps", type=int, default=200,
                    help="decode steps of the official layer leg (T=2048 runs 5)")
    ap.add_argument("--no-official", action="store_true")
    ap.add_argument("--no-storage", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the GPU legs of configs 1, 2 and 4")
    ap.add_argument("--cpu-quick", action="store_true",
                    help="CPU baseline on configs 1-3 only (by default also config 4 in full "
                         "at N threads, one thread on a 1/16 token sample, and a labelled "
                         "1/16 token sample of config 5)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="short workload for a rocprofv3 --pmc pass: a 256 MiB device copy "
                         "(counter calibration), then decode layer calls")
    ap.add_argument("--pmc-prefill", action="store_true",
                    help="short workload for a rocprofv3 --pmc pass over the T=2048 prefill "
                         "chunk: the calibration copy, then --steps prefill layer calls")
    ap.add_argument("--pmc-c4", action="store_true",
                    help="short workload for a rocprofv3 --pmc pass over the T=64 "
                         "verification window (config 4's Zipf-skewed router on one bank): "
                         "the calibration copy, then --steps layer calls on one stream")
    ap.add_argument("--scaled-fp4", action="store_true",
                    help="with --pmc-prefill: the routed experts on the scaled FP4 MFMA "
                         "(K3X_FLAG_SCALED_FP4)")
    ap.add_argument("--counters-from", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc passes over one of the --pmc-* workloads "
                         "(per-kernel medians, HBM bytes from FETCH_SIZE / WRITE_SIZE against "
                         "the calibration copy, the memory-unit busy share) into "
                         "--counters-out")
    ap.add_argument("--counters-out", default=os.path.join("profiles", "prefill_c5_counters.json"),
                    help="JSON file (relative to the repo root) --counters-from writes")
    ap.add_argument("--counters-workload", default="bench.py --pmc-prefill (c5 prefill chunk, "
                    "T=2048, one stream)", help="workload named in the --counters-out file")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn the FETCH_SIZE and WRITE_SIZE pass outputs into " + TRAFFIC_JSON_REL)
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.traffic_from:
        print(json.dumps(traffic_from(*args.traffic_from)))
        return 0
    if args.counters_from:
        print(json.dumps(counters_from(args.counters_from, args.counters_out,
                                       args.counters_workload)))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the layer and its resident "
                                   "bank live on a single MI355X (--gpus 1)",
                          "n_gpus": args.gpus}))
        return 2
    import numpy as np
    import torch
    import k3x_amd

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs an MI355X (no HIP device visible)")
    dev = "cuda:0"
    ctx = k3x_amd.Context(0)
    shape = k3x_amd.LayerShape(H, I, E, S)
    banks = []
    for layer in range(args.layers):
        b = k3x_amd.Bank(ctx, shape)
        b.fill_synthetic(SEED + layer, SCALE_LO, SCALE_HI, 0.02, 0.1, 0.02, 1.0)
        banks.append(b)
    log(f"{args.layers} banks resident, {banks[0].bytes() / 1e9:.2f} GB each")

    T = 2
    xs = []
    for i in range(args.inputs):
        x = torch.empty((T, H), dtype=torch.int16, device=dev)
        k3x_amd.synth_normal_bf16(ctx, X_SEED + i, k3x_amd.stream_id(k3x_amd.STREAM_INPUT), 1.0, x)
        xs.append(x)
    out = torch.empty((T, H), dtype=torch.int16, device=dev)
    params = k3x_amd.make_params(T, K, 2.5, 1e-6, k3x_amd.GLU_SWIGLU, 4.0, None,
                                 k3x_amd.RENORM_FLOAT)
    combos = np.lcm(args.layers, args.inputs)
    if args.pmc_prefill:
        src = torch.empty(CALIB_BYTES // 4, dtype=torch.int32, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # the calibration copy: reads and writes CALIB_BYTES
        torch.cuda.synchronize()
        Tp = 2048
        xp = torch.empty((Tp, H), dtype=torch.int16, device=dev)
        k3x_amd.synth_normal_bf16(ctx, X_SEED + 1000, k3x_amd.stream_id(k3x_amd.STREAM_INPUT),
                                  1.0, xp)
        outp = torch.empty((Tp, H), dtype=torch.int16, device=dev)
        pp = k3x_amd.make_params(Tp, K, 2.5, 1e-6, k3x_amd.GLU_SWIGLU, 4.0, None,
                                 k3x_amd.RENORM_FLOAT,
                                 k3x_amd.FLAG_SCALED_FP4 if args.scaled_fp4 else 0)
        ctx.set_profiling(True)  # one stream: every kernel in stream order, no overlap
        for i in range(max(args.steps, 1)):
            k3x_amd.check(k3x_amd.moe_forward(ctx, banks[0], pp, xp, outp), "prefill")
            k3x_amd.check(ctx.synchronize(), "pmc prefill")
        for b in banks:
            b.close()
        ctx.close()
        log("pmc prefill pass done")
        return 0
    if args.pmc_c4:
        src = torch.empty(CALIB_BYTES // 4, dtype=torch.int32, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # the calibration copy: reads and writes CALIB_BYTES
        torch.cuda.synchronize()
        sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]
        from oracle import Oracle
        from synth import CONFIGS, SynthLayer
        cfg = CONFIGS[4]
        layer = SynthLayer(Oracle(), cfg)
        k3x_amd.check(banks[0].upload_router(layer.router, layer.bias, layer.gamma), "c4 router")
        x4 = torch.empty((cfg.tokens, H), dtype=torch.int16, device=dev)
        k3x_amd.synth_normal_bf16(ctx, cfg.x_seed, k3x_amd.stream_id(k3x_amd.STREAM_INPUT), 1.0,
                                  x4)
        out4 = torch.empty((cfg.tokens, H), dtype=torch.int16, device=dev)
        p4 = k3x_amd.make_params(cfg.tokens, cfg.top_k, cfg.routed_scale, cfg.eps, cfg.glu,
                                 cfg.beta, cfg.linear, cfg.renorm)
        ctx.set_profiling(True)  # one stream: every kernel in stream order, no overlap
        for i in range(max(args.steps, 1)):
            k3x_amd.check(k3x_amd.moe_forward(ctx, banks[0], p4, x4, out4), "c4")
            k3x_amd.check(ctx.synchronize(), "pmc c4")
        for b in banks:
            b.close()
        ctx.close()
        log("pmc c4 pass done")
        return 0
    if args.pmc_pass:
        src = torch.empty(CALIB_BYTES // 4, dtype=torch.int32, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # the calibration copy: reads and writes CALIB_BYTES
        torch.cuda.synchronize()
        for i in range(max(args.steps, 8)):
            k3x_amd.check(k3x_amd.moe_forward(ctx, banks[i % args.layers], params,
                                              xs[i % args.inputs], out), "moe_forward")
        k3x_amd.check(ctx.synchronize(), "pmc pass")
        for b in banks:
            b.close()
        ctx.close()
        log("pmc pass done")
        return 0

    # Distinct experts each (layer, input) call touches, for the byte count.
    active = {}
    na = torch.empty(1, dtype=torch.int32, device=dev)
    for i in range(combos):
        lb, xi = i % args.layers, i % args.inputs
        k3x_amd.check(k3x_amd.moe_forward(ctx, banks[lb], params, xs[xi], out,
                                          {"n_active": na}), "moe_forward")
        k3x_amd.check(ctx.synchronize(), "synchronize")
        active[(lb, xi)] = int(na.item())
    touched = [active[(i % args.layers, i % args.inputs)] for i in range(combos)]
    mean_d = sum(touched) / len(touched)

    def step(i: int) -> None:
        st = k3x_amd.moe_forward(ctx, banks[i % args.layers], params, xs[i % args.inputs], out)
        if st:
            raise k3x_amd.K3xError(st, "moe_forward")

    def run(n: int) -> float:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n):
            step(i)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    # The read-ceiling leg (its own figure, below) runs first: 4 GiB streamed
    # 23 times brings the device to its loaded clock before the warm-up steps,
    # which a short run (20 steps after 5) would otherwise spend inside.
    ceiling = read_ceiling(ctx, k3x_amd, torch)
    run(args.warmup)
    k3x_amd.check(ctx.synchronize(), "warmup")
    log(f"timing {args.steps} steps")
    elapsed = run(args.steps)
    k3x_amd.check(ctx.synchronize(), "timed steps")
    us = elapsed / args.steps * 1e6

    # The same number of steps on the device's own clock: hipEvents on the
    # layer's stream around steps 2 .. K + 1 of a run of K + 1, so that the
    # host's start-up (the first call's submission after the synchronisation,
    # which the wall clock above includes) is not in the interval.
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    step(0)
    ev0.record()
    for i in range(1, args.steps + 1):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    event_us = ev0.elapsed_time(ev1) * 1e3 / args.steps
    k3x_amd.check(ctx.synchronize(), "event-timed steps")

    # Same steps again with per-stage hipEvent pairs on the layer's stream.
    ctx.set_profiling(True)
    ctx.stage_times(reset=True)
    prof_elapsed = run(args.steps)
    stages = ctx.stage_times(reset=True)
    ctx.set_profiling(False)
    k3x_amd.check(ctx.synchronize(), "profiled steps")

    routed_bytes = mean_d * EXPERT_BYTES
    all_bytes = routed_bytes + SHARED_GU_BYTES + SHARED_DOWN_BYTES + ROUTER_BYTES + 2 * T * H * 2
    stage_bytes = {
        "gate_up": mean_d * GATE_UP_BYTES + T * H * 2,
        "down": mean_d * DOWN_BYTES,
        "shared_gate_up": SHARED_GU_BYTES,
        "shared_down": SHARED_DOWN_BYTES,
        "route": ROUTER_BYTES + T * H * 2,
        # decode path: front = router + shared gate/up blocks; select =
        # Top-K block + shared down blocks.
        "decode_front": ROUTER_BYTES + SHARED_GU_BYTES + T * H * 2,
        "decode_select": SHARED_DOWN_BYTES,
        "decode_gate_up": mean_d * GATE_UP_BYTES + T * H * 2,
        "decode_down": mean_d * DOWN_BYTES,
    }
    stage_report = {}
    for name, (ms, n) in stages.items():
        if not n:
            continue
        avg_us = ms / n * 1e3
        entry = {"avg_us": round(avg_us, 3), "launches": int(n)}
        if name in stage_bytes:
            entry["gbps"] = round(stage_bytes[name] / (avg_us * 1e-6) / 1e9, 1)
        stage_report[name] = entry
    dom = max(("gate_up", "down", "shared_gate_up", "shared_down", "decode_front",
               "decode_select", "decode_gate_up", "decode_down"),
              key=lambda s: stage_report.get(s, {}).get("avg_us", 0.0))
    dom_us = stage_report[dom]["avg_us"]
    achieved = stage_bytes[dom] / (dom_us * 1e-6) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, TRAFFIC_JSON_REL)
    if os.path.exists(tpath):
        with open(tpath) as f:
            kern = json.load(f)["kernels"].get(STAGE_KERNEL.get(dom, ""))
        if kern:
            traffic = kern["hbm_bytes_per_dispatch"]

    result = {
        "metric": "MoE-layer µs @T=2 decode (HBM GB/s, %peak); MXFP4 TFLOPS @T=2048",
        "value": round(us, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded generator; random-init weights of the K3 layer shape)",
        "config": {"workload": "c3_decode_layer: T=2, H=7168, E=384 MXFP4 experts I=2048, "
                               "Top-16 sigmoid+bias router x2.5, bf16 shared expert I=2048, "
                               "RMSNorm, device routing",
                   "tokens": T, "layers_cycled": args.layers, "inputs_cycled": args.inputs},
        "tokens_per_s": round(T / (us * 1e-6), 1),
        "experts_touched_mean": mean_d,
        "hbm_gbps_routed": round(routed_bytes / (us * 1e-6) / 1e9, 1),
        "hbm_frac_routed": round(routed_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "hbm_gbps_all": round(all_bytes / (us * 1e-6) / 1e9, 1),
        "hbm_frac_all": round(all_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "profiled_us_per_layer": round(prof_elapsed / args.steps * 1e6, 3),
        "event_us_per_layer": round(event_us, 3),
        "stages": stage_report,
        "roofline": {"bound": "hbm", "kernel": dom,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": round(stage_bytes[dom]),
                     "traffic_source": TRAFFIC_JSON_REL if traffic else None},
    }
    result["roofline"]["read_ceiling"] = ceiling
    result["roofline"]["frac_of_read_ceiling"] = round(achieved / ceiling["gbps"], 4)

    if not args.no_prefill:
        result["prefill"] = prefill(args, ctx, banks[0], k3x_amd, torch)
    if not args.no_configs:
        result["configs"] = config_legs(ctx, banks[0], k3x_amd, torch)
    for b in banks:
        b.close()
    if not args.no_official:
        result["official"] = official(args, ctx, k3x_amd, torch)
    if not args.no_storage:
        result["storage"] = storage(ctx, k3x_amd, torch, cpu=not args.no_cpu_baseline)
    if not args.no_cpu_baseline:
        result["cpu_baseline"], result["cpu_configs"] = cpu_baseline(not args.cpu_quick)
    ctx.close()
    print(json.dumps(result), flush=True)
    return 0


def read_ceiling(ctx, k3x_amd, torch) -> dict:
    """The device's plain streaming-read rate (k3x_hip_stream_read over 4 GiB
    resident in HBM, 20 calls back to back): the practical ceiling a
    streaming kernel's rate is read against, beside the nominal 8 TB/s."""
    n, calls = 4 << 30, 20
    buf = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    fold = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    for _ in range(3):
        k3x_amd.check(ctx.stream_read(buf, fold), "stream_read")
    k3x_amd.check(ctx.synchronize(), "synchronize")
    t0 = time.perf_counter()
    for _ in range(calls):
        k3x_amd.check(ctx.stream_read(buf, fold), "stream_read")
    k3x_amd.check(ctx.synchronize(), "synchronize")
    dt = (time.perf_counter() - t0) / calls
    del buf
    return {"gbps": round(n / dt / 1e9, 1), "bytes": n, "calls": calls,
            "frac_of_peak": round(n / dt / 1e9 / HBM_PEAK_GBS, 4),
            "kernel": "stream_read_kernel (k3x_hip_stream_read)"}


def prefill(args, ctx, bank, k3x_amd, torch) -> dict:
    """T=2048 tokens through the same layer shape."""
    T = 2048
    dev = "cuda:0"
    x = torch.empty((T, H), dtype=torch.int16, device=dev)
    k3x_amd.synth_normal_bf16(ctx, X_SEED + 1000, k3x_amd.stream_id(k3x_amd.STREAM_INPUT), 1.0, x)
    out = torch.empty((T, H), dtype=torch.int16, device=dev)
    na = torch.empty(1, dtype=torch.int32, device=dev)
    params = k3x_amd.make_params(T, K, 2.5, 1e-6, k3x_amd.GLU_SWIGLU, 4.0, None,
                                 k3x_amd.RENORM_FLOAT)
    k3x_amd.check(k3x_amd.moe_forward(ctx, bank, params, x, out, {"n_active": na}), "prefill")
    k3x_amd.check(ctx.synchronize(), "prefill")
    d = int(na.item())

    def timed(p) -> float:
        k3x_amd.check(k3x_amd.moe_forward(ctx, bank, p, x, out), "prefill")  # warm scratch
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.prefill_steps):
            k3x_amd.check(k3x_amd.moe_forward(ctx, bank, p, x, out), "prefill")
        torch.cuda.synchronize()
        k3x_amd.check(ctx.synchronize(), "prefill")
        return (time.perf_counter() - t0) / args.prefill_steps * 1e6

    us = timed(params)
    # The same chunk with the routed experts on the scaled FP4 MFMA.
    scaled = k3x_amd.make_params(T, K, 2.5, 1e-6, k3x_amd.GLU_SWIGLU, 4.0, None,
                                 k3x_amd.RENORM_FLOAT, k3x_amd.FLAG_SCALED_FP4)
    us_scaled = timed(scaled)
    log(f"prefill T=2048, scaled FP4 MFMA: {us_scaled:.1f} us/layer")
    routed_flops = T * K * EXPERT_FLOPS
    all_flops = routed_flops + T * SHARED_FLOPS
    bytes_ = d * EXPERT_BYTES + SHARED_GU_BYTES + SHARED_DOWN_BYTES + ROUTER_BYTES + 2 * T * H * 2
    tflops = routed_flops / (us * 1e-6) / 1e12
    floor_us = max(bytes_ / (HBM_PEAK_GBS * 1e9), routed_flops / (MXFP4_PEAK_TFLOPS * 1e12)) * 1e6
    log(f"prefill T=2048: {us:.1f} us/layer")
    return {"workload": "c5_prefill_chunk: T=2048, same layer", "tokens": T,
            "steps": args.prefill_steps, "us_per_layer": round(us, 1),
            "tokens_per_s": round(T / (us * 1e-6), 1), "experts_touched": d,
            "routed_tflops": round(tflops, 2),
            "all_tflops": round(all_flops / (us * 1e-6) / 1e12, 2),
            "mxfp4_peak_frac": round(tflops / MXFP4_PEAK_TFLOPS, 4),
            "hbm_frac": round(bytes_ / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "roofline_floor_us": round(floor_us, 1),
            "frac_of_floor": round(floor_us / us, 4),
            "scaled_fp4": {"flags": "K3X_FLAG_SCALED_FP4", "us_per_layer": round(us_scaled, 1),
                           "tokens_per_s": round(T / (us_scaled * 1e-6), 1),
                           "routed_tflops": round(routed_flops / (us_scaled * 1e-6) / 1e12, 2)}}


def time_calls(torch, fn, n: int, warmup: int = 3) -> float:
    """Microseconds per call of fn(i) over n calls after `warmup` untimed ones,
    bracketed by device synchronisation."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / n * 1e6


def config_legs(ctx, bank_c3, k3x_amd, torch) -> dict:
    """The other benchmark configurations through the same entry point
    (k3x_hip_moe_forward, device routing), each timed over whole layer calls
    with inputs resident in HBM:
    c1  the tiny layer (T=1, H=256, E=16, I=512, Top-4), 8 banks cycled;
    c2  one K3-shaped expert (T=1, H=7168, I=2048, E=1, Top-1, no shared
        expert), 32 banks cycled so no cache holds the 23.4 MB expert;
    c4  the verification window (T=64, Zipf-skewed bias over the c3 bank,
        0..~40 rows per expert; the general path's narrow GEMMs)."""
    sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]
    from oracle import Oracle
    from synth import CONFIGS, SynthLayer
    dev = "cuda:0"
    out = {}
    na = torch.empty(1, dtype=torch.int32, device=dev)
    for cid, nbanks, steps in ((1, 8, 400), (2, 32, 400), (4, 1, 20)):
        cfg = CONFIGS[cid]
        T, Hc, Ic, Ec, Kc, Sc = (cfg.tokens, cfg.hidden, cfg.inter, cfg.experts, cfg.top_k,
                                 cfg.shared_inter)
        if cid == 4:
            layer = SynthLayer(Oracle(), cfg)
            k3x_amd.check(bank_c3.upload_router(layer.router, layer.bias, layer.gamma),
                          "c4 router")
            banks = [bank_c3]
        else:
            banks = []
            for i in range(nbanks):
                b = k3x_amd.Bank(ctx, k3x_amd.LayerShape(Hc, Ic, Ec, Sc))
                b.fill_synthetic(cfg.seed + i, cfg.scale_lo, cfg.scale_hi, cfg.router_sigma,
                                 cfg.bias_sigma, cfg.shared_sigma, 1.0)
                banks.append(b)
        x = torch.empty((T, Hc), dtype=torch.int16, device=dev)
        k3x_amd.synth_normal_bf16(ctx, cfg.x_seed, k3x_amd.stream_id(k3x_amd.STREAM_INPUT), 1.0,
                                  x)
        y = torch.empty((T, Hc), dtype=torch.int16, device=dev)
        params = k3x_amd.make_params(T, Kc, cfg.routed_scale, cfg.eps, cfg.glu, cfg.beta,
                                     cfg.linear, cfg.renorm)
        k3x_amd.check(k3x_amd.moe_forward(ctx, banks[0], params, x, y, {"n_active": na}),
                      f"c{cid}")
        k3x_amd.check(ctx.synchronize(), f"c{cid}")
        d = int(na.item())

        def call(i):
            st = k3x_amd.moe_forward(ctx, banks[i % len(banks)], params, x, y)
            if st:
                raise k3x_amd.K3xError(st, f"c{cid}")

        us = time_calls(torch, call, steps)
        k3x_amd.check(ctx.synchronize(), f"c{cid}")
        expert_bytes = 3 * (Hc * Ic // 2 + Hc * Ic // 32)
        routed = d * expert_bytes
        all_b = routed + 3 * Sc * Hc * 2 + Ec * Hc * 4 + Ec * 4 + Hc * 4 + 2 * T * Hc * 2
        flops = T * Kc * 2 * 3 * Hc * Ic + T * 2 * 3 * Hc * Sc
        out[f"c{cid}"] = {
            "workload": cfg.name, "tokens": T, "hidden": Hc, "inter": Ic, "experts": Ec,
            "top_k": Kc, "shared_inter": Sc, "banks_cycled": len(banks), "steps": steps,
            "us_per_layer": round(us, 2), "tokens_per_s": round(T / (us * 1e-6), 1),
            "experts_touched": d, "routed_bytes": routed,
            "hbm_gbps_routed": round(routed / (us * 1e-6) / 1e9, 1),
            "hbm_frac_routed": round(routed / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "hbm_gbps_all": round(all_b / (us * 1e-6) / 1e9, 1),
            "tflops": round(flops / (us * 1e-6) / 1e12, 3)}
        log(f"c{cid}: {us:.1f} us/layer, {d} experts touched")
        if cid != 4:
            for b in banks:
                b.close()
    return out


# The official K3 MoE FFN (Stable LatentMoE): hidden 7168, latent 3584, 896
# MXFP4 experts of 3072 at the latent width, Top-16, bf16 shared FFN of 6144.
OH, OL, OI, OE, OK, OS = 7168, 3584, 3072, 896, 16, 6144
O_EXPERT_BYTES = 3 * (OL * OI // 2 + OL * OI // 32)                 # 17,547,264
O_DENSE_BYTES = 2 * OL * OH * 2 + 3 * OS * OH * 2                   # routed down/up + shared
O_ROUTE_BYTES = OE * OH * 4 + OE * 4 + 3 * OH * 4 + OL * 4          # router, vectors


def official(args, ctx, k3x_amd, torch) -> dict:
    """The official layer at its own shapes: prepare (two-source mix, router
    logits) + FFN (route, latent projection, experts, routed_norm, routed_up,
    shared FFN, output) per step, on synthetic weights; T=2 decode and a
    T=2048 prefill chunk."""
    dev = "cuda:0"
    bank = k3x_amd.Bank(ctx, k3x_amd.LayerShape(OL, OI, OE, 0))
    bank.fill_synthetic(SEED + 100, SCALE_LO, SCALE_HI, 0.02, 0.1, 0.02, 1.0)
    off = k3x_amd.Official(ctx, bank, OH, OS)
    off.fill_synthetic(SEED + 101, 0.02, 0.02, 0.05, 0.1)
    out = {"workload": "official K3 MoE FFN: H=7168, latent 3584, E=896 MXFP4 experts of "
                       "I=3072, Top-16, shared FFN 6144; prepare + FFN per step",
           "data": "synthetic weights and inputs"}
    for T, n in ((2, args.official_steps), (2048, 5)):
        g = torch.Generator(device=dev)
        g.manual_seed(T)
        prefix = torch.randn((T, OH), device=dev, generator=g)
        residual = torch.randn((T, OH), device=dev, generator=g)
        hidden = torch.empty((T, OH), dtype=torch.int16, device=dev)
        y = torch.empty((T, OH), dtype=torch.int16, device=dev)
        ids = torch.empty((T, OK), dtype=torch.int32, device=dev)
        params = k3x_amd.make_params(T, OK, 1.0, 1e-5, k3x_amd.GLU_SITU, 4.0, 25.0,
                                     k3x_amd.RENORM_DOUBLE)

        def step(taps=None):
            k3x_amd.check(off.prepare(T, 1e-5, prefix, residual, hidden), "official prepare")
            k3x_amd.check(off.ffn(params, hidden, prefix, y, taps=taps), "official ffn")

        step({"ids": ids})
        for _ in range(3):
            step()
        k3x_amd.check(ctx.synchronize(), "official")
        touched = int(torch.unique(ids).numel())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            step()
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) / n * 1e6
        k3x_amd.check(ctx.synchronize(), "official")
        bytes_ = touched * O_EXPERT_BYTES + O_DENSE_BYTES + O_ROUTE_BYTES + 4 * T * OH * 4
        flops = T * (OK * 2 * 3 * OL * OI + 2 * (2 * OL * OH + 3 * OS * OH) + 2 * OE * OH)
        key = "decode_t2" if T == 2 else "prefill_t2048"
        out[key] = {"tokens": T, "steps": n, "us_per_layer": round(us, 1),
                    "experts_touched": touched, "bytes": bytes_,
                    "hbm_gbps": round(bytes_ / (us * 1e-6) / 1e9, 1),
                    "hbm_frac": round(bytes_ / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                    "tflops": round(flops / (us * 1e-6) / 1e12, 2)}
        log(f"official T={T}: {us:.1f} us/layer ({touched} experts)")
    off.close()
    bank.close()
    return out


def storage(ctx, k3x_amd, torch, cpu: bool) -> dict:
    """K3X storage records: the device CRC32C over 256 MiB resident in HBM, and
    load_storage_expert of official-shape experts (3 x 3072 x 3584 MXFP4,
    17,547,264 B) from a K3X file in the page cache into bank slots (read into
    pinned memory, one H2D copy, six CRC32C checks on the device, re-tile)."""
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from golden.k3x_fixture import expert_tensors, write_k3x
    dev = "cuda:0"
    n = 256 << 20
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    buf = torch.randint(0, 256, (n,), dtype=torch.uint8, device=dev, generator=g)
    k3x_amd.check(ctx.crc32c(buf)[0], "crc32c")
    reps = 10
    t0 = time.perf_counter()
    for _ in range(reps):
        k3x_amd.check(ctx.crc32c(buf)[0], "crc32c")
    crc_s = (time.perf_counter() - t0) / reps
    out = {"crc32c": {"bytes": n, "us_per_call": round(crc_s * 1e6, 1),
                      "gbps": round(n / crc_s / 1e9, 1),
                      "hbm_frac": round(n / crc_s / 1e9 / HBM_PEAK_GBS, 4),
                      "note": "whole call: kernel, 64 Ki chunk values to the host, host fold"}}
    del buf

    def dcrc(b: bytes) -> int:
        t = torch.frombuffer(bytearray(b), dtype=torch.uint8).to(dev)
        st, c = ctx.crc32c(t, len(b))
        k3x_amd.check(st, "crc32c")
        return c

    L, I, E = OL, OI, 8
    rng = torch.Generator().manual_seed(11)
    tensors = []
    for e in range(E):
        ex = {f"{r}_packed": torch.randint(0, 256, (I * L // 2,), dtype=torch.uint8,
                                           generator=rng).numpy()
              for r in ("gate", "up", "down")}
        ex.update({f"{r}_scales": torch.randint(119, 124, (I * L // 32,), dtype=torch.uint8,
                                                generator=rng).numpy()
                   for r in ("gate", "up", "down")})
        tensors += expert_tensors(1, e, ex, I, L)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "experts.k3x")
        write_k3x(path, tensors, dcrc)
        bank = k3x_amd.Bank(ctx, k3x_amd.LayerShape(L, I, E, 0))
        store = k3x_amd.Storage(path)
        k3x_amd.check(store.open_status, "storage open")
        for e in range(E):  # warm: page cache, pinned and device staging
            k3x_amd.check(store.upload_expert(bank, e, 1, e)[0], "storage upload")
        passes = 3
        t0 = time.perf_counter()
        for _ in range(passes):
            for e in range(E):
                st, nbytes = store.upload_expert(bank, e, 1, e)
                k3x_amd.check(st, "storage upload")
        per = (time.perf_counter() - t0) / (passes * E)
        store.close()
        bank.close()
    out["expert_load"] = {"expert_bytes": nbytes, "experts": E, "passes": passes,
                          "us_per_expert": round(per * 1e6, 1),
                          "gbps": round(nbytes / per / 1e9, 2),
                          "source": "K3X file in the page cache"}
    if cpu:
        # The reference's byte-table CRC32C (runtime/src/crc32c.cpp), restated
        # by the oracle and pinned to it (tests/test_oracle_vs_ref.py), single
        # thread, on 64 MiB of the same kind of data.
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        from oracle import Oracle
        data = torch.randint(0, 256, (64 << 20,), dtype=torch.uint8, generator=rng).numpy()
        o = Oracle()
        t0 = time.perf_counter()
        o.crc32c_table(data)
        cpu_s = time.perf_counter() - t0
        out["crc32c"]["cpu_baseline"] = {"value": round(data.size / cpu_s / 1e9, 3),
                                         "unit": "GB/s", "cores": 1, "kind": "port",
                                         "sample": "64 MiB, k3xo_crc32c_table (the byte-table "
                                                   "method of runtime/src/crc32c.cpp)"}
    log(f"storage: crc32c {out['crc32c']['gbps']} GB/s, expert load "
        f"{out['expert_load']['us_per_expert']} us")
    return out


def traffic_from(fetch_dir: str, write_dir: str) -> dict:
    """Per-dispatch HBM bytes of each decode kernel from two rocprofv3 --pmc
    passes over `bench.py --pmc-pass` (FETCH_SIZE, then WRITE_SIZE, KiB per
    dispatch), each scaled by what the same counter reads for the pass's
    plain CALIB_BYTES device copy.  Writes TRAFFIC_JSON_REL."""
    import csv
    import glob
    import statistics

    def read(d: str, counter: str) -> dict:
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            raise SystemExit(f"no counter_collection.csv under {d}")
        per = {}
        for fn in files:
            with open(fn) as f:
                for r in csv.DictReader(f):
                    if r["Counter_Name"] != counter:
                        continue
                    name = r["Kernel_Name"]
                    key = next((k for k in set(STAGE_KERNEL.values()) if k in name), None)
                    if key is None and "copyBuffer" in name:
                        key = "calibration_copy"
                    if key:
                        per.setdefault(key, []).append(float(r["Counter_Value"]))
        return per

    fetch, write = read(fetch_dir, "FETCH_SIZE"), read(write_dir, "WRITE_SIZE")
    # The calibration copy is the largest copyBuffer dispatch of the pass.
    cf, cw = max(fetch["calibration_copy"]), max(write["calibration_copy"])
    kf, kw = CALIB_BYTES / (cf * 1024), CALIB_BYTES / (cw * 1024)
    kernels = {}
    for k in sorted(set(fetch) & set(write) - {"calibration_copy"}):
        mf, mw = statistics.median(fetch[k]), statistics.median(write[k])
        kernels[k] = {"dispatches": len(fetch[k]), "fetch_kib_median": round(mf, 1),
                      "write_kib_median": round(mw, 1),
                      "hbm_bytes_per_dispatch": round(mf * 1024 * kf + mw * 1024 * kw)}
    out = {"workload": "bench.py --pmc-pass (c3 decode layer, T=2, banks cycled)",
           "commands": ["rocprofv3 --pmc FETCH_SIZE --output-format csv -d <FETCH_DIR> -o run -- "
                        "python3 bench.py --pmc-pass --steps 64",
                        "rocprofv3 --pmc WRITE_SIZE --output-format csv -d <WRITE_DIR> -o run -- "
                        "python3 bench.py --pmc-pass --steps 64",
                        "python3 bench.py --traffic-from <FETCH_DIR> <WRITE_DIR>"],
           "calibration": {"copy_bytes": CALIB_BYTES, "fetch_kib": cf, "write_kib": cw,
                           "fetch_scale": round(kf, 4), "write_scale": round(kw, 4)},
           "kernels": kernels}
    with open(os.path.join(ROOT, TRAFFIC_JSON_REL), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    return out


COUNTERS_JSON_REL = os.path.join("profiles", "prefill_c5_counters.json")
XCD_COUNT = 8  # MI355X: GRBM_GUI_ACTIVE reports DIMENSION_XCC[0:7], summed


def counters_from(dirs: list[str], out_rel: str = COUNTERS_JSON_REL,
                  workload: str = "bench.py --pmc-prefill (c5 prefill chunk, T=2048, one stream)"
                  ) -> dict:
    """Per-kernel medians of every counter in rocprofv3 --pmc passes over one
    of the --pmc-* workloads (one directory per pass), with HBM bytes per
    dispatch from FETCH_SIZE / WRITE_SIZE scaled by the calibration copy, for
    the MFMA kernels the MFMA-busy share of the busy cycles, and the memory
    unit's busy share (TA_BUSY_avr over the per-XCD GRBM_GUI_ACTIVE: the
    texture addresser, which every vector memory instruction passes; the
    MemUnitBusy of earlier profilers).  Writes out_rel."""
    import csv
    import glob
    import re
    import statistics

    per: dict = {}
    calib: dict = {}
    for d in dirs:
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            raise SystemExit(f"no counter_collection.csv under {d}")
        for fn in files:
            with open(fn) as f:
                for r in csv.DictReader(f):
                    name, c, v = r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"])
                    if "copyBuffer" in name:
                        calib[c] = max(calib.get(c, 0.0), v)
                        continue
                    m = re.search(r"(\w+)(<[^()]*>)?\(", name.replace("(anonymous namespace)::", ""))
                    key = (m.group(1) + (m.group(2) or "")) if m else name
                    per.setdefault(key, {}).setdefault(c, []).append(v)
    kf = CALIB_BYTES / (calib["FETCH_SIZE"] * 1024) if "FETCH_SIZE" in calib else None
    kw = CALIB_BYTES / (calib["WRITE_SIZE"] * 1024) if "WRITE_SIZE" in calib else None
    kernels = {}
    for k, cs in sorted(per.items()):
        row = {"dispatches": max(len(v) for v in cs.values())}
        for c, vals in sorted(cs.items()):
            row[c] = round(statistics.median(vals), 1)
        if kf and kw and "FETCH_SIZE" in cs and "WRITE_SIZE" in cs:
            row["hbm_bytes_per_dispatch"] = round(row["FETCH_SIZE"] * 1024 * kf +
                                                  row["WRITE_SIZE"] * 1024 * kw)
        if cs.get("SQ_BUSY_CYCLES") and cs.get("SQ_VALU_MFMA_BUSY_CYCLES"):
            row["mfma_busy_over_sq_busy"] = round(row["SQ_VALU_MFMA_BUSY_CYCLES"] /
                                                  max(row["SQ_BUSY_CYCLES"], 1.0), 4)
        mops = sum(row.get(f"SQ_INSTS_VALU_MFMA_MOPS_{t}", 0.0) for t in ("BF16", "F8", "F6F4", "F64"))
        if mops:
            # Each MOPS unit is 512 floating-point operations.
            row["mfma_tflop_issued_per_dispatch"] = round(mops * 512 / 1e12, 4)
        if cs.get("TA_BUSY_avr") and cs.get("GRBM_GUI_ACTIVE"):
            # GRBM_GUI_ACTIVE is summed over the XCDs' instances; the TA
            # average is per TA, so per-XCD active cycles divide it.
            row["mem_unit_busy_pct"] = round(100.0 * row["TA_BUSY_avr"] * XCD_COUNT /
                                             max(row["GRBM_GUI_ACTIVE"], 1.0), 1)
        kernels[k] = row
    out = {"workload": workload,
           "calibration": {"copy_bytes": CALIB_BYTES, **calib,
                           "fetch_scale": round(kf, 4) if kf else None,
                           "write_scale": round(kw, 4) if kw else None},
           "kernels": kernels}
    with open(os.path.join(ROOT, out_rel), "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    return out


def cpu_threads() -> int:
    """Threads for the N-thread CPU baseline: the CPU share this process may
    use (OMP_NUM_THREADS when the host sets it, else the affinity mask)."""
    env = os.environ.get("OMP_NUM_THREADS")
    n = len(os.sched_getaffinity(0))
    return max(1, min(int(env), n)) if env and env.isdigit() else n


def cpu_baseline(all_configs: bool) -> tuple[dict, dict]:
    """The reference's CPU expert path, restated by the oracle (k3x_oracle.c,
    k3xo_moe_layer: pinned bit for bit to the reference's own CPU composition
    by tests/test_oracle_vs_ref.py), timed on this host: rms_norm -> router
    (double sums) -> libm sigmoid + bias Top-K -> per (token, slot) pair the
    MXFP4 expert (decode to fp32, double GEMVs, GLU) -> slot-ordered mix +
    bf16 shared expert.  One thread (the reference backend is
    single-threaded) and N threads over tokens and pairs.  Returns the
    headline entry (config 3 at N threads) and the per-config table."""
    import numpy as np
    sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]
    from oracle import ORDER_SEQ, SIGMOID_REF, Oracle, bf16_to_f32
    from synth import CONFIGS, SynthLayer

    o = Oracle()
    n_thr = cpu_threads()
    table = {"threads_n": n_thr, "nproc": os.cpu_count(), "kind": "port",
             "source": "oracle/k3x_oracle.c k3xo_moe_layer"}

    def run(cid, tokens=None, threads=(1, n_thr)):
        cfg = CONFIGS[cid]
        layer = SynthLayer(o, cfg)
        x = bf16_to_f32(layer.x_bits())
        if tokens is not None:
            x = x[tokens]
        T = x.shape[0]
        # The experts the routes reach (the same double-sum router and libm
        # sigmoid as the timed call), generated on the host.
        need = set()
        for t in range(T):
            xn = o.rms_norm(x[t], layer.gamma, cfg.eps)
            st, ids, _, _ = o.route(o.router_logits(layer.router, xn, ORDER_SEQ), layer.bias,
                                    cfg.top_k, cfg.renorm, cfg.routed_scale, SIGMOID_REF)
            need |= {int(e) for e in ids}
        layer.prefetch(need, n_thr)
        experts = [layer.expert(e) if e in need else None for e in range(cfg.experts)]
        row = {"tokens": T, "pairs": T * cfg.top_k, "experts_touched": len(need)}
        for n in threads:
            t0 = time.perf_counter()
            st, _, _, _ = o.moe_layer(x, layer.gamma, cfg.eps, layer.router, layer.bias,
                                      experts, cfg.hidden, cfg.inter, cfg.top_k,
                                      cfg.routed_scale, cfg.renorm, layer.shared, cfg.glu,
                                      cfg.beta, cfg.linear, threads=n)
            sec = time.perf_counter() - t0
            if st:
                raise RuntimeError(f"CPU layer c{cid} failed: {st}")
            row[f"us_{n}thr"] = round(sec * 1e6, 1)
        log(f"cpu c{cid} ({T} tokens): " + ", ".join(f"{k} {v}" for k, v in row.items()))
        return row

    for cid in (1, 2, 3):
        table[f"c{cid}"] = run(cid)
        table[f"c{cid}"]["sample"] = "full layer call"
    if all_configs:
        # Config 4 in full at N threads (one thread on every 16th token,
        # x16); config 5 on every 16th token at N threads (x16, labelled
        # derived).
        table["c4"] = run(4, threads=(n_thr,))
        table["c4"]["sample"] = "full layer call, N threads"
        sub = run(4, tokens=list(range(0, 64, 16)), threads=(1,))
        table["c4"]["us_1thr"] = round(sub["us_1thr"] * 16, 1)
        table["c4"]["us_1thr_derived_from"] = "4 of 64 tokens (every 16th), x16"
        c5 = run(5, tokens=list(range(0, 2048, 16)), threads=(n_thr,))
        table["c5"] = {"tokens": 2048, "derived": True,
                       f"us_{n_thr}thr": round(c5[f"us_{n_thr}thr"] * 16, 1),
                       "sample": "128 of 2048 tokens (every 16th), N threads, x16",
                       "sample_experts_touched": c5["experts_touched"]}
    c3 = table["c3"]
    head = {"value": c3[f"us_{n_thr}thr"], "unit": "us/layer", "cores": n_thr, "kind": "port",
            "value_1thr": c3["us_1thr"],
            "sample": "one full config-3 layer call (T=2: RMSNorm, router, Top-16, 32 routed "
                      "pairs, shared expert) through k3xo_moe_layer, the oracle's pinned "
                      f"restatement of the reference CPU path, {n_thr} threads; value_1thr "
                      "is the same call on one thread"}
    return head, table


if __name__ == "__main__":
    sys.exit(main())
