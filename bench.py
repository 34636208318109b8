#!/usr/bin/env python3
"""Benchmark of the MI355X backend for tt-lab's quantized decode path.

Prints ONE JSON line (see the fields below).  One GPU only: --gpus N with N > 1
exits with a message.

Workload: one gpt-oss-20b MoE layer at decode batch 1 --
router 32x2880 (bf16 values in f32), top-4 + softmax, per selected expert MXFP4
gate/up 2x2880x2880 with the clamped SwiGLU, MXFP4 down 2880x2880, weighted
combine.  24 distinct synthetic layers (10.2 GB of experts) are resident and a step
runs one token through all 24 in a HIP graph, so weights stream from HBM rather
than the 256 MB Infinity Cache.

roofline: the fused gate/up+SwiGLU kernel (the largest of the layer), timed live
with HIP events around a graph of back-to-back launches over the 24 layers.
cpu_baseline: the CPU oracle's restatement of the reference's v4 (AVX-512) body,
one thread, on a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tt-lab_amd"))

METRIC = "decode tok/s at gpt-oss-20b shape; MXFP4 matvec GB/s and % of HBM peak"
N = 2880
EXPERTS, USED, LAYERS = 32, 4, 24
HBM_PEAK_GBS = 8000.0
# Algorithmic bytes of one gate/up+SwiGLU launch: 4 experts x (gate + up) x 2880 rows x
# 1530 B, their f32 biases, x (f32 2880) read, hidden (f32 4x2880) written.
GATEUP_BYTES = USED * 2 * N * 1530 + USED * 2 * N * 4 + N * 4 + USED * N * 4
# Algorithmic bytes of one token-layer (config 1): bf16 router, 4 x (gate+up+down) MXFP4,
# x in, out, routing.
LAYER_BYTES = EXPERTS * N * 2 + USED * 3 * N * 1530 + N * 4 + N * 4 + 128


def log(msg):
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def build_layers(dev, ttlab_amd):
    layers = []
    for l in range(LAYERS):
        seed = 0x77000100 + l
        gate = dev.mxfp4_synthetic(N, N, EXPERTS, seed, 1000)
        up = dev.mxfp4_synthetic(N, N, EXPERTS, seed, 2000)
        down = dev.mxfp4_synthetic(N, N, EXPERTS, seed, 3000)
        rw = dev.alloc(EXPERTS * N * 4)
        dev.synth_normal_bf16(rw, seed, 20, EXPERTS * N, 0.02)
        rb = dev.alloc(EXPERTS * 4)
        dev.fill(rb, 0)
        x = dev.alloc(N * 4)
        dev.synth_normal(x, 0x78000100 + l, 0, N)
        d = ttlab_amd.MoeLayerDesc()
        d.hidden, d.expert_hidden, d.experts, d.used = N, N, EXPERTS, USED
        d.router_weight, d.router_bias = rw.ptr, rb.ptr
        d.gate, d.up, d.down = gate.handle, up.handle, down.handle
        d.gate_bias = d.up_bias = d.down_bias = None
        layers.append({"desc": d, "x": x, "out": dev.alloc(N * 4), "idx": dev.alloc(64), "w": dev.alloc(64),
                       "hidden": dev.alloc(USED * N * 4), "keep": (gate, up, down, rw, rb)})
    dev.sync()
    return layers


def gpu_run(args):
    import ttlab_amd

    dev = ttlab_amd.Device(0)
    info = dev.info()
    log(f"device {info}")
    layers = build_layers(dev, ttlab_amd)
    log(f"{LAYERS} layers resident")

    def step():
        for L in layers:
            dev.moe_decode(L["desc"], L["x"], L["out"], L["idx"], L["w"])

    graph = dev.capture(step)
    for _ in range(max(args.warmup, 1)):
        graph.launch()
    dev.sync()
    dev.timer_start()
    for _ in range(args.steps):
        graph.launch()
    ms = dev.timer_stop()
    ms_per_step = ms / args.steps
    token_layers_per_s = LAYERS / (ms_per_step * 1e-3)
    log(f"{ms_per_step:.4f} ms per step ({LAYERS} token-layers), {token_layers_per_s:.0f} token-layers/s")

    # Dominant kernel: gate/up + SwiGLU over the 24 layers, indices from the routing above.
    def gateup():
        for L in layers:
            dev.moe_gateup_swiglu(L["desc"], L["x"], L["idx"], L["hidden"])

    g2 = dev.capture(gateup)
    for _ in range(3):
        g2.launch()
    dev.sync()
    reps = max(20, args.steps)
    dev.timer_start()
    for _ in range(reps):
        g2.launch()
    ms2 = dev.timer_stop()
    launch_us = ms2 * 1e3 / (reps * LAYERS)
    achieved = GATEUP_BYTES / (launch_us * 1e-6) / 1e9
    log(f"gateup_swiglu_kernel: {launch_us:.2f} us per launch, {achieved:.0f} GB/s")
    layer_gbs = LAYER_BYTES * token_layers_per_s / 1e9
    graph.free()
    g2.free()
    dev.close()
    return {
        "ms_per_step": ms_per_step,
        "value": token_layers_per_s,
        "layer_gbs": layer_gbs,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gateup_swiglu_kernel", "bytes_per_launch": GATEUP_BYTES,
                     "launch_us": round(launch_us, 3)},
        "device": info,
    }


def cpu_baseline(seconds):
    """Oracle (restated reference v4 body) on one host core, bounded sample of config 1."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import ctypes as C

    import numpy as np

    import oracle_lib as O
    from moe_fixtures import HostLayer

    try:
        os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    except OSError:
        pass
    host = HostLayer(EXPERTS, USED, biases=False, seed=0x77000100)
    body = O.BODY_V4_SIMD if O.has_avx512() else O.BODY_V4
    out = np.empty(N, np.float32)
    s = host.oracle_struct()
    xs = [O.synth_normal(0x78000200, t, N) for t in range(16)]
    count, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        O.lib.orc_moe(C.byref(s), xs[count % 16], out, body, None, None, None)
        count += 1
    elapsed = time.perf_counter() - t0
    isa = "AVX-512 (x86-64-v4 body)" if body == O.BODY_V4_SIMD else "x86-64-v3 (v4 body restated with fmaf)"
    return {"value": round(count / elapsed, 3), "unit": "token-layers/s", "cores": 1, "kind": "port",
            "sample": f"{count} token-layers of config 1 (one 32-expert layer, 16 distinct x) in {elapsed:.1f} s; "
                      f"oracle restatement of tensor.cpp v4 matvec + model.cpp moe; {isa}"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    res = gpu_run(args)
    base = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(res["value"], 1),
        "unit": "token-layers/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (MXFP4 weights)",
        "data": "synthetic",
        "config": {"workload": "config 1: gpt-oss-20b MoE layer, decode batch 1; step = one token through "
                               "24 distinct resident layers (HIP graph)",
                   "experts": EXPERTS, "used": USED, "hidden": N, "layers_per_step": LAYERS,
                   "layer_algorithmic_GBps": round(res["layer_gbs"], 1)},
        "roofline": res["roofline"],
        "cpu_baseline": base,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
