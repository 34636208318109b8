#!/usr/bin/env python3
"""Benchmark of the MI355X backend for tt-lab's quantized decode path.

Prints ONE JSON line.  One GPU only: --gpus N with N > 1 exits with a message.

Default workload: full synthetic gpt-oss-20b decode at
batch 1 -- 24 layers, 64 q / 8 kv heads of 64, sinks, sliding window 128 on even
layers, 32 experts top-4 MXFP4, vocab 201088 bf16 unembedding, greedy.  The KV
caches are first filled to 2048 positions by running the decode itself; then a
step is one token through the whole model (one HIP graph replay, the token fed
back on the device) and value = tokens/s.

roofline: the MXFP4 gate/up + SwiGLU expert kernel (the path's dominant kernel),
timed live with HIP events around a graph of the 24 layers' launches; bytes per
launch are the 4 selected experts' gate and up rows, their biases, x and the
SwiGLU output.  The line's
"matvec" field is config 0 (one 5760x2880 MXFP4 matvec over 1.13 GB of rotated
matrices), measured in the same run: the metric's "MXFP4 matvec GB/s".  The
line's "other_configs" field holds configs 1, 2 (bf16 and scaled paths) and 4 from
the same run, each its own workload below with fewer steps (--no-other-configs
skips them).

cpu_baseline: the CPU oracle's restatement of the reference's forward
(model.cpp:557-602) on one host core, over a bounded sample: one sliding-window
layer and one full-context layer at position 2048 plus the unembedding; a token
is 12 of each plus the unembedding.

--workload moe runs benchmark config 1 instead: one MoE layer per step over 24
distinct resident layers, value = token-layers/s.

--workload prefill runs benchmark config 2: the batched prefill experts of one MoE
layer for 512 bf16 tokens with balanced given routing (bf16 MFMA, the down GEMM
on f16 MFMA over the hidden's two f16 planes where the down weights' E8M0 scales
keep their f16 decode exact; with --activations mxfp8 the scaled fp8 x fp4 MFMA
path), value = token-layers/s;
roofline on the larger of the gate/up and down GEMM launches.

--workload model-prefill runs the full synthetic gpt-oss-20b model's layer-major
prefill (GptOssModel::prefill) of a 512-token prompt, value = prompt tokens/s;
roofline = the pass's algorithmic MFMA rate (2 x active weights x tokens).
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
EXPERTS, USED, LAYERS, VOCAB, CONTEXT = 32, 4, 24, 201088, 2048
HBM_PEAK_GBS = 8000.0
SEED = 0x77000003
# Algorithmic bytes of one gate/up+SwiGLU launch: 4 experts x (gate + up) x 2880 rows x
# 1530 B, their f32 biases, x (f32 2880) read, hidden (f32 4x2880) written.
GATEUP_BYTES = USED * 2 * N * 1530 + USED * 2 * N * 4 + N * 4 + USED * N * 4
# Algorithmic bytes of the step's one-launch gate/up + down: the 4 experts' gate, up and
# down rows and biases, x, and the down outputs (the hidden stays inside the launch).
GATEUP_DOWN_BYTES = USED * 3 * N * 1530 + USED * 3 * N * 4 + N * 4 + USED * N * 4
Q8_ROW_2880, Q8_ROW_4096 = 90 * 34, 128 * 34
# The committed rocprofv3 summary the measured HBM bytes per launch come from
# (FETCH_SIZE and WRITE_SIZE runs, scaled on a known-size copy).
HBM_BYTES_PROFILE = os.path.join(ROOT, "profiles", "decode_cfg3_hbm_bytes.txt")


def measured_traffic(kernel):
    """HBM bytes per dispatch of `kernel` (its name as rocprofv3 prints it) from the
    committed counter summary, or None if the summary has no line for it."""
    try:
        with open(HBM_BYTES_PROFILE) as f:
            for line in f:
                if line.startswith("  ") and line.strip().startswith(kernel) and "total" in line:
                    return int(round(float(line.split("total")[1].split()[0]) * 1e6))
    except OSError:
        pass
    return None


def step_kernel_bytes(kind, position, experts, vocab):
    """Algorithmic bytes one launch of a decode-step kernel must move: the weights and
    cache entries the reference's arithmetic reads, its f32 inputs and outputs."""
    span_full = position + 1
    if kind == "qkv":  # Q8_0 5120 x 2880; the previous layer's residual, 4 down outputs and
        # weights (the combine staged in), norm; bias, q out, k/v out, one RoPE row
        return 5120 * Q8_ROW_2880 + (2 + USED) * N * 4 + 5120 * 4 + 4096 * 4 + 2 * 512 * 4 + 64 * 4
    if kind in ("attention_window", "attention_full"):  # K and V of the span, q, out, sinks
        span = min(span_full, 128) if kind == "attention_window" else span_full
        return 2 * span * 512 * 4 + 2 * 4096 * 4 + 64 * 4
    if kind == "output":  # Q8_0 2880 x 4096, attended, bias, residual in, out
        return N * Q8_ROW_4096 + 4096 * 4 + 3 * N * 4
    if kind == "router_rows":  # f32 router, bias, x, norm
        return experts * N * 4 + experts * 4 + 2 * N * 4
    if kind in ("gateup_routed", "gateup_given"):
        return GATEUP_BYTES
    if kind == "gateup_down":
        return GATEUP_DOWN_BYTES
    if kind == "down":  # 4 experts' down rows and biases, hidden in, 4 outputs
        return USED * N * 1530 + 3 * USED * N * 4
    if kind == "logits":  # bf16 unembedding; residual, 4 down outputs, norm; logits out
        return vocab * N * 2 + (2 + USED) * N * 4 + vocab * 4
    raise ValueError(kind)


def log(msg):
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def read_ceiling(nbytes, buffers, reps=20):
    """Microseconds per launch of a plain streaming read (ttl_stream_read) of nbytes,
    over `buffers` distinct buffers replayed as one graph: the fixed launch cost and
    the streaming rate this chip gives a kernel that only reads, at the same bytes
    per launch as the measured kernel."""
    import ctypes as C

    import ttlab_amd

    dev = ttlab_amd.Device(0)
    bufs = [dev.alloc(nbytes) for _ in range(buffers)]
    for b in bufs:
        dev.fill(b, 0x5a)
    sink = dev.alloc(256)

    def launches():
        for b in bufs:
            ttlab_amd._check(dev.lib.ttl_stream_read(dev.ctx, b.ptr, nbytes, sink.ptr), "ttl_stream_read")

    g = dev.capture(launches)
    for _ in range(3):
        g.launch()
    dev.sync()
    dev.timer_start()
    for _ in range(reps):
        g.launch()
    us = 1e3 * dev.timer_stop() / (reps * buffers)
    g.free()
    for b in bufs + [sink]:
        b.free()
    dev.close()
    return us


def ceiling_entry(achieved_gbs, nbytes, us_read):
    gbs = nbytes / (us_read * 1e-6) / 1e9
    return {"kernel": "stream_read_kernel (plain 16-byte loads, no arithmetic)", "bytes_per_launch": nbytes,
            "launch_us": round(us_read, 3), "GBps": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "kernel_frac_of_ceiling": round(achieved_gbs / gbs, 4)}


def gpu_decode(args):
    import ttlab_amd

    context, experts = args.context, args.experts
    capacity = context + args.warmup + args.steps + 8
    t0 = time.time()
    model = ttlab_amd.Model(args.layers, experts, VOCAB, capacity, SEED)
    if args.eager:
        model.set_graph_replay(False)
    model_bytes = model.device_bytes
    log(f"model resident: {model_bytes / 1e9:.2f} GB in {time.time() - t0:.1f} s")
    t0 = time.time()
    if args.kv_fill == "synthetic":
        model.fill_kv_synthetic(context)
        token = 1
        log(f"KV caches filled to {context} positions with synthetic values ({time.time() - t0:.1f} s)")
    else:
        filled = model.generate(1, 0, context)
        log(f"KV caches filled to {context} positions by decoding ({time.time() - t0:.1f} s)")
        token = int(filled[-1])
    ms = model.time_decode(token, context, args.warmup, args.steps)
    tok_s = 1000.0 / ms
    mid = context + args.warmup + args.steps // 2
    step_bytes = model.step_bytes(mid)
    log(f"{ms:.4f} ms per token, {tok_s:.1f} tok/s, step {step_bytes / 1e9:.3f} GB -> "
        f"{step_bytes / (ms * 1e-3) / 1e9:.0f} GB/s algorithmic")
    # every kind of the step's kernels, timed one kind at a time at the last step's position
    last = context + args.warmup + args.steps - 1
    reps = max(20, args.steps // 5)
    kernels, total_us = {}, 0.0
    for kind in ttlab_amd.Model.KERNELS:
        us_k, n = model.time_kernel(kind, last, reps)
        if n == 0:  # e.g. no full-context layer in a one-layer counter run
            continue
        nbytes = step_kernel_bytes(kind, last, experts, VOCAB)
        gbs = nbytes / (us_k * 1e-6) / 1e9
        kernels[kind] = {"us": round(us_k, 3), "launches_per_step": n, "bytes_per_launch": nbytes,
                         "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        # the step runs gate/up with its ranking (routed) and down as two launches; gate/up
        # with the indices given and the one-launch gate/up + down are timed for comparison
        if kind not in ("gateup_given", "gateup_down"):
            total_us += us_k * n
        log(f"{kind:17s} {n:3d} launches x {us_k:7.2f} us, {gbs:7.0f} GB/s ({gbs / HBM_PEAK_GBS:.3f} of peak)")
    log(f"sum of the step's kernels timed one kind at a time: {total_us / 1000:.4f} ms (step {ms:.4f} ms)")
    us = kernels["gateup_routed"]["us"]
    achieved = GATEUP_BYTES / (us * 1e-6) / 1e9
    model.close()
    us_read = read_ceiling(GATEUP_BYTES, args.layers)
    log(f"plain read of the same {GATEUP_BYTES / 1e6:.1f} MB per launch: {us_read:.2f} us, "
        f"{GATEUP_BYTES / (us_read * 1e-6) / 1e9:.0f} GB/s")
    given, fused = kernels["gateup_given"], kernels["gateup_down"]
    if args.table:
        write_table(args.table, args, ms, step_bytes, kernels, total_us, us_read)
    # the metric's second half: config 0's standalone MXFP4 matvec, in the same run
    matvec = None
    if not getattr(args, "skip_matvec", False):
        mv_us, mv_gbs, mv_read = measure_matvec(args)
        matvec = {"workload": MATVEC_WORKLOAD, "kernel": "matvec_kernel", "bytes_per_launch": MATVEC_BYTES,
                  "launch_us": round(mv_us, 3), "GBps": round(mv_gbs, 1), "frac": round(mv_gbs / HBM_PEAK_GBS, 4),
                  "read_ceiling": ceiling_entry(mv_gbs, MATVEC_BYTES, mv_read)}
    return {
        "matvec": matvec,
        "value": tok_s,
        "unit": "tok/s",
        "ms_per_step": ms,
        "config": {"workload": f"config {args.config}: full synthetic gpt-oss-{'20b' if args.config == 3 else '120b'} "
                               f"decode, batch 1, greedy, KV context {context} (filled by decoding), step = one token "
                               "(one HIP graph replay)",
                   "layers": args.layers, "experts": experts, "experts_used": USED, "vocab": VOCAB,
                   "device_GB": round(model_bytes / 1e9, 2),
                   "context": context, "unembedding": "bf16", "attention_weights": "Q8_0",
                   "step_algorithmic_bytes": int(step_bytes),
                   "step_algorithmic_GBps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                   "step_frac_of_hbm_peak": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "kernels": kernels,
                   "kernels_sum_ms": round(total_us / 1000, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     # the committed counters are config 3's (PL = 1: at most 64 experts)
                     "traffic": measured_traffic("void gateup_swiglu_kernel<0, true, 1>") if args.config == 3 else None,
                     "kernel": f"gateup_swiglu_kernel<0, true, {1 if experts <= 64 else 2 if experts <= 128 else 3}> "
                               "(top-4 ranking at its head, then gate/up of the 4 experts and the clamped SwiGLU, "
                               "on the router rows' normalized input; as the step runs it)",
                     "bytes_per_launch": GATEUP_BYTES, "launch_us": round(us, 3),
                     "given_indices": {"kernel": "gateup_swiglu_kernel<1, false, 3>", "launch_us": given["us"],
                                       "GBps": given["GBps"], "frac": given["frac"]},
                     "one_launch_with_down": {"kernel": "gateup_down_kernel<0, true, 1> (not the step's: level with "
                                                        "the two launches alone, slower in the step)",
                                              "bytes_per_launch": GATEUP_DOWN_BYTES, "launch_us": fused["us"],
                                              "GBps": fused["GBps"], "frac": fused["frac"]},
                     "read_ceiling": ceiling_entry(achieved, GATEUP_BYTES, us_read)},
    }


def write_table(path, args, ms, step_bytes, kernels, total_us, us_read):
    """The decode run's per-kind kernel table (HIP events around graph replays of every
    launch of one kind in a step), as text, for committing beside a rocprof summary
    of the same invocation."""
    mode = "eager launches" if args.eager else "graph replays"
    lines = [f"# bench.py per-kind decode kernel table (HIP events, {mode}): config {args.config}, "
             f"{args.layers} layers, KV context {args.context}",
             f"#   command: python3 bench.py {' '.join(sys.argv[1:])}",
             f"#   step: {ms:.4f} ms per token, {1000.0 / ms:.1f} tok/s, {step_bytes / 1e9:.3f} GB algorithmic",
             f"# {'kind':17s} {'launches':>8s} {'us':>8s} {'bytes':>12s} {'GB/s':>8s} {'frac':>7s}"]
    for kind, k in kernels.items():
        lines.append(f"  {kind:17s} {k['launches_per_step']:8d} {k['us']:8.3f} {k['bytes_per_launch']:12d} "
                     f"{k['GBps']:8.1f} {k['frac']:7.4f}")
    lines.append(f"# sum of the step's kernels (gateup_given and gateup_down, timed for comparison, excluded): "
                 f"{total_us / 1000:.4f} ms")
    lines.append(f"# stream_read_kernel of {GATEUP_BYTES} B (the gate/up launch's bytes): {us_read:.3f} us")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def gpu_moe(args):
    import ttlab_amd

    dev = ttlab_amd.Device(0)
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
        layers.append({"desc": d, "x": x, "out": dev.alloc(N * 4), "idx": dev.alloc(64), "w": dev.alloc(64),
                       "hidden": dev.alloc(USED * N * 4), "keep": (gate, up, down, rw, rb)})
    dev.sync()

    def step():
        for L in layers:
            dev.moe_decode(L["desc"], L["x"], L["out"], L["idx"], L["w"])

    def gateup():
        for L in layers:
            dev.moe_gateup_swiglu(L["desc"], L["x"], L["idx"], L["hidden"])

    # --eager launches one by one (for kernel tracers that do not follow graph launches)
    graph = None if args.eager else dev.capture(step)
    run = step if args.eager else graph.launch
    for _ in range(max(args.warmup, 1)):
        run()
    dev.sync()
    dev.timer_start()
    for _ in range(args.steps):
        run()
    ms = dev.timer_stop() / args.steps

    g2 = None if args.eager else dev.capture(gateup)
    run2 = gateup if args.eager else g2.launch
    for _ in range(3):
        run2()
    dev.sync()
    reps = max(20, args.steps)
    dev.timer_start()
    for _ in range(reps):
        run2()
    us = dev.timer_stop() * 1e3 / (reps * LAYERS)
    achieved = GATEUP_BYTES / (us * 1e-6) / 1e9
    for g in (graph, g2):
        if g:
            g.free()
    dev.close()
    layer_bytes = EXPERTS * N * 2 + USED * 3 * N * 1530 + N * 4 + N * 4 + 128
    return {
        "value": LAYERS / (ms * 1e-3),
        "unit": "token-layers/s",
        "ms_per_step": ms,
        "config": {"workload": "config 1: gpt-oss-20b MoE layer, decode batch 1; step = one token through 24 "
                               "distinct resident layers (HIP graph)",
                   "experts": EXPERTS, "used": USED, "hidden": N, "layers_per_step": LAYERS,
                   "layer_algorithmic_GBps": round(layer_bytes * LAYERS / (ms * 1e-3) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("void gateup_swiglu_kernel<0, false, 3>"),
                     "kernel": "gateup_swiglu_kernel<0, false, 3> (indices given)", "bytes_per_launch": GATEUP_BYTES,
                     "launch_us": round(us, 3)},
    }


# Config 0: y = W x for the 5760 x 2880 MXFP4 matrix (gate and up stacked: the GGUF
# {2880, 2880, 2} bytes are the same rows in the same order as one 5760-row matrix),
# one ttl_matvec_mxfp4 launch.  The copies are distinct resident matrices replayed in
# rotation, 1.13 GB in all (four times the 256 MB MALL), so every launch streams its
# weights from HBM.
MATVEC_COPIES = 128
MATVEC_BYTES = 2 * N * 1530 + N * 4 + 2 * N * 4  # W, x, y: 8,847,360
MATVEC_FLOP = 2 * 2 * N * N


def measure_matvec(args):
    """Config 0 on the device: microseconds per launch of one 5760x2880 MXFP4 matvec over
    MATVEC_COPIES distinct resident matrices replayed in rotation (1.13 GB, beyond every
    cache), and of a plain read of the same bytes per launch."""
    import ttlab_amd

    dev = ttlab_amd.Device(0)
    mats = [dev.mxfp4_synthetic(2 * N, N, 1, 0x77000000, 100 + i) for i in range(MATVEC_COPIES)]
    x = dev.alloc(N * 4)
    dev.synth_normal(x, 0x78000000, 0, N)
    y = dev.alloc(2 * N * 4)
    dev.sync()

    def step():
        for w in mats:
            dev.matvec_mxfp4(w, None, x, y, 0)

    # --eager launches one by one (for kernel tracers that do not follow graph launches)
    graph = None if args.eager else dev.capture(step)
    run = step if args.eager else graph.launch
    for _ in range(max(args.warmup, 1)):
        run()
    dev.sync()
    reps = max(20, args.steps)
    dev.timer_start()
    for _ in range(reps):
        run()
    ms = dev.timer_stop()
    us = ms * 1e3 / (reps * MATVEC_COPIES)
    gbs = MATVEC_BYTES / (us * 1e-6) / 1e9
    log(f"config 0 matvec: {us:.3f} us per launch, {gbs:.0f} GB/s over {MATVEC_COPIES} rotated copies")
    if graph:
        graph.free()
    for w in mats:
        w.free()
    for b in (x, y):
        b.free()
    dev.close()
    us_read = read_ceiling(MATVEC_BYTES, MATVEC_COPIES)
    log(f"plain read of the same {MATVEC_BYTES / 1e6:.2f} MB per launch: {us_read:.2f} us, "
        f"{MATVEC_BYTES / (us_read * 1e-6) / 1e9:.0f} GB/s")
    return us, gbs, us_read


MATVEC_WORKLOAD = ("config 0: one 5760x2880 MXFP4 matvec (gate|up stacked) per launch; "
                   f"{MATVEC_COPIES} distinct resident matrices (1.13 GB) replayed in rotation; step = one launch")


def gpu_matvec(args):
    us, gbs, us_read = measure_matvec(args)
    return {
        "value": gbs,
        "unit": "GB/s",
        "ms_per_step": us * 1e-3,
        "config": {"workload": MATVEC_WORKLOAD,
                   "rows": 2 * N, "cols": N, "bytes_per_launch": MATVEC_BYTES,
                   "matvec_GFLOPs": round(MATVEC_FLOP / (us * 1e-6) / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "matvec_kernel", "bytes_per_launch": MATVEC_BYTES, "launch_us": round(us, 3),
                     "read_ceiling": ceiling_entry(gbs, MATVEC_BYTES, us_read)},
    }


PREFILL_TOKENS = 512
PREFILL_LAYERS = 3  # distinct resident layers (1.27 GB of experts, beyond every cache)
PREFILL_PAIRS = PREFILL_TOKENS * USED
# Algorithmic bytes and flops of the two GEMM launches of one config-2 layer:
# gate/up reads all 32 experts' gate and up rows, the bf16 activations of the 512
# tokens, and writes the f32 hidden of the 2048 (token, expert) pairs; down reads
# the down rows and that hidden and writes the f32 down outputs.
PF_GATEUP_BYTES = EXPERTS * 2 * N * 1530 + PREFILL_TOKENS * N * 2 + PREFILL_PAIRS * N * 4
PF_DOWN_BYTES = EXPERTS * N * 1530 + 2 * PREFILL_PAIRS * N * 4
PF_GATEUP_FLOP = 2 * 2 * PREFILL_PAIRS * N * N
PF_DOWN_FLOP = 2 * PREFILL_PAIRS * N * N
MFMA_BF16_PEAK_TFLOPS = 2500.0
# The scaled path (--activations mxfp8) moves MXFP8 instead of bf16/f32 activations:
# one byte per element plus one E8M0 byte per 32.  Gate/up reads the tokens' MXFP8
# activations and writes the pairs' MXFP8 hidden; down reads that hidden and writes
# the f32 down outputs.  Its MFMA peak is the fp8 one (the mixed fp4 x fp8 operands
# run at the fp8 rate).
MX8_ROW = N + N // 32
PF_MX8_GATEUP_BYTES = EXPERTS * 2 * N * 1530 + PREFILL_TOKENS * MX8_ROW + PREFILL_PAIRS * MX8_ROW
PF_MX8_DOWN_BYTES = EXPERTS * N * 1530 + PREFILL_PAIRS * MX8_ROW + PREFILL_PAIRS * N * 4
MFMA_FP8_PEAK_TFLOPS = 5000.0


def gpu_prefill(args):
    import numpy as np

    import ttlab_amd

    dev = ttlab_amd.Device(0)
    keep, descs = [], []
    for l in range(PREFILL_LAYERS):
        seed = 0x77000300 + l
        gate = dev.mxfp4_synthetic(N, N, EXPERTS, seed, 1000)
        up = dev.mxfp4_synthetic(N, N, EXPERTS, seed, 2000)
        down = dev.mxfp4_synthetic(N, N, EXPERTS, seed, 3000)
        d = ttlab_amd.MoeLayerDesc()
        d.hidden, d.expert_hidden, d.experts, d.used = N, N, EXPERTS, USED
        d.gate, d.up, d.down = gate.handle, up.handle, down.handle
        keep += [gate, up, down]
        descs.append(d)
    # the down GEMM runs on the hidden's two f16 planes when every down expert's scales allow
    hidden_f16 = all(t.f16_exact for t in keep[2::3])
    xs = np.random.RandomState(0x78000002).randn(PREFILL_TOKENS * N).astype(np.float32)
    x = dev.upload(ttlab_amd.bf16_bits(xs))
    idx, w = ttlab_amd.balanced_routing(PREFILL_TOKENS, EXPERTS, USED, 0x79000002)
    ib, wb = dev.upload(idx), dev.upload(w)
    out = dev.alloc(PREFILL_TOKENS * N * 4)
    scaled = args.activations == "mxfp8"
    dt = ttlab_amd.TTL_DTYPE_BF16_AS_MXFP8 if scaled else ttlab_amd.TTL_DTYPE_BF16
    ws = dev.alloc(dev.moe_prefill_workspace_bytes(PREFILL_TOKENS, EXPERTS, USED, dt))

    def run(stages, layers):
        def fn():
            for d in layers:
                dev.moe_prefill_experts(d, x, dt, PREFILL_TOKENS, ib, wb, out, ws, stages)
        return fn

    def time_graph(fn, launches, reps):
        g = dev.capture(fn)
        for _ in range(3):
            g.launch()
        dev.sync()
        dev.timer_start()
        for _ in range(reps):
            g.launch()
        ms = dev.timer_stop() / (reps * launches)
        g.free()
        return ms

    ms = time_graph(run(ttlab_amd.TTL_PREFILL_ALL, descs), PREFILL_LAYERS, max(1, args.steps // PREFILL_LAYERS))
    # the two GEMM launches alone (the plan and fragments stay in the workspace)
    reps = max(10, args.steps // (2 * PREFILL_LAYERS))
    us_gu = 1e3 * time_graph(run(ttlab_amd.TTL_PREFILL_GATEUP, descs * 2), 2 * PREFILL_LAYERS, reps)
    us_dn = 1e3 * time_graph(run(ttlab_amd.TTL_PREFILL_DOWN, descs * 2), 2 * PREFILL_LAYERS, reps)
    dev.sync()
    for b in (x, ib, wb, out, ws):
        b.free()
    for t in keep:
        t.free()
    dev.close()
    log(f"prefill layer: {ms * 1e3:.1f} us ({PREFILL_TOKENS / ms * 1e3:.0f} token-layers/s); gate/up "
        f"{us_gu:.1f} us, down {us_dn:.1f} us")
    if scaled:
        kernels = {
            "mx8_gateup_kernel": (us_gu, PF_MX8_GATEUP_BYTES, PF_GATEUP_FLOP),
            "mx8_matmul_kernel (down)": (us_dn, PF_MX8_DOWN_BYTES, PF_DOWN_FLOP),
        }
    else:
        kernels = {
            "gateup_kernel": (us_gu, PF_GATEUP_BYTES, PF_GATEUP_FLOP),
            "matmul_kernel (down)": (us_dn, PF_DOWN_BYTES, PF_DOWN_FLOP),
        }
    name = max(kernels, key=lambda k: kernels[k][0])
    us, nbytes, flop = kernels[name]
    achieved = nbytes / (us * 1e-6) / 1e9
    us_read = read_ceiling(nbytes, 2 * PREFILL_LAYERS)
    log(f"plain read of the same {nbytes / 1e6:.1f} MB per launch: {us_read:.2f} us, "
        f"{nbytes / (us_read * 1e-6) / 1e9:.0f} GB/s")
    per_kernel = {k: {"us": round(v[0], 2), "algorithmic_GBps": round(v[1] / (v[0] * 1e-6) / 1e9, 1),
                      "algorithmic_TFLOPs": round(v[2] / (v[0] * 1e-6) / 1e12, 1)} for k, v in kernels.items()}
    return {
        "value": PREFILL_TOKENS / (ms * 1e-3),
        "unit": "token-layers/s",
        "ms_per_step": ms,
        "dtype": ("MXFP8 activations and hidden x MXFP4 weights, f32 accumulate (scaled fp8/fp4 MFMA)" if scaled
                  else "bf16 activations x MXFP4 weights, f32 accumulate (bf16 MFMA; down on f16 MFMA over "
                       "the hidden's two f16 planes)" if hidden_f16
                  else "bf16 activations x MXFP4 weights, f32 accumulate (bf16 MFMA; down over the hidden's "
                       "three bf16 planes)"),
        "config": {"workload": "config 2: batched prefill experts of one gpt-oss-20b MoE layer, 512 bf16 tokens, "
                               "top-4 of 32 experts, balanced given routing (64 tokens per expert); step = one layer "
                               f"(plan, gather, gate/up+SwiGLU, down, combine) over {PREFILL_LAYERS} distinct "
                               "resident layers (HIP graph)",
                   "activations": args.activations,
                   "tokens": PREFILL_TOKENS, "experts": EXPERTS, "used": USED, "hidden": N,
                   "kernels": per_kernel},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": name,
                     "bytes_per_launch": nbytes, "launch_us": round(us, 3),
                     "mfma_algorithmic_TFLOPs": round(flop / (us * 1e-6) / 1e12, 1),
                     "mfma_peak_TFLOPs": MFMA_FP8_PEAK_TFLOPS if scaled else MFMA_BF16_PEAK_TFLOPS,
                     "read_ceiling": ceiling_entry(achieved, nbytes, us_read)},
    }


PROMPT_TOKENS = 512
# Multiply-adds per token and layer of the prefill pass: 4 experts x 3 matrices of
# 2880 x 2880, the Q/K/V (5120 x 2880) and output (2880 x 4096) projections, the router.
PREFILL_MACS_PER_TOKEN_LAYER = USED * 3 * N * N + 5120 * N + N * 4096 + EXPERTS * N


def gpu_model_prefill(args):
    import numpy as np

    import ttlab_amd

    t0 = time.time()
    model = ttlab_amd.Model(args.layers, args.experts, VOCAB, PROMPT_TOKENS + 16, SEED)
    log(f"model resident: {model.device_bytes / 1e9:.2f} GB in {time.time() - t0:.1f} s")
    tokens = [int(t) for t in np.random.default_rng(0x79000010).integers(0, VOCAB, PROMPT_TOKENS)]
    for _ in range(max(1, min(args.warmup, 3))):
        model.prefill(tokens)
    reps = max(3, args.steps // 20)
    t0 = time.perf_counter()
    for _ in range(reps):
        model.prefill(tokens)
    ms = (time.perf_counter() - t0) / reps * 1e3
    model.close()
    flop = 2.0 * PREFILL_MACS_PER_TOKEN_LAYER * PROMPT_TOKENS * args.layers
    tflops = flop / (ms * 1e-3) / 1e12
    log(f"prefill of {PROMPT_TOKENS} tokens: {ms:.2f} ms, {PROMPT_TOKENS / ms * 1e3:.0f} tok/s, "
        f"{tflops:.0f} TFLOP/s algorithmic")
    return {
        "value": PROMPT_TOKENS / (ms * 1e-3),
        "unit": "prompt tok/s",
        "ms_per_step": ms,
        "dtype": "f16 MFMA, f32 accumulate: f32 activations (and the SwiGLU hidden) as two f16 planes "
                 "scaled by a power of two per token, exact weights (three exact bf16 planes on bf16 MFMA "
                 "where MXFP4 scales leave the f16 range)",
        "config": {"workload": f"full synthetic gpt-oss-{'20b' if args.config == 3 else '120b'} layer-major prefill "
                               f"of a {PROMPT_TOKENS}-token prompt (GptOssModel::prefill); step = one prefill "
                               "(host tokens in, last-token logits out)",
                   "layers": args.layers, "experts": args.experts, "tokens": PROMPT_TOKENS,
                   "algorithmic_TFLOP_per_step": round(flop / 1e12, 3)},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": "whole prefill pass (MoE and Q8_0 GEMMs, attention, norms)",
                     "flop_per_step": flop},
    }


def host_cpu():
    """Model name, online cores and the x86 ISA extensions that matter to the oracle."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    isa = [f for f in ("avx2", "fma", "f16c", "avx512f", "avx512bw", "avx512vl", "avx512_vnni") if f in flags]
    # allowed_cores: the cores this process may run on; the sample itself uses one
    return {"model": model, "nproc": os.cpu_count(), "allowed_cores": len(os.sched_getaffinity(0)), "isa": isa}


def cpu_baseline(seconds, workload, layers=LAYERS, context=CONTEXT):
    """The oracle (restated reference CPU path) on one host core, bounded sample."""
    host = host_cpu()  # before the sample pins this process to one core
    res = _cpu_baseline(seconds, workload, layers, context)
    res["host"] = host
    return res


def _cpu_baseline(seconds, workload, layers=LAYERS, context=CONTEXT):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import ctypes as C

    import numpy as np

    import oracle_lib as O

    try:
        os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    except OSError:
        pass
    body = O.BODY_V4_SIMD if O.has_avx512() else O.BODY_V4
    isa = "AVX-512 (x86-64-v4 body)" if body == O.BODY_V4_SIMD else "x86-64-v3 (v4 body restated with fmaf)"
    if workload == "prefill":
        from moe_fixtures import HostLayer

        # one expert's share of a config-2 layer: 64 tokens through its gate, up and down
        # (selected-token matmuls, model.cpp:404-447), times the 32 experts
        host = HostLayer(1, 1, biases=False, seed=0x77000300)
        s = host.oracle_struct()
        tokens = 64
        x = O.synth_normal_bf16(0x78000002, 0, tokens * N, 1.0)
        idx = np.zeros(tokens, np.int64)
        w = np.ones(tokens, np.float32)
        out = np.empty(tokens * N, np.float32)
        count, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds or count == 0:
            O.lib.orc_moe_batch_experts(C.byref(s), x, tokens, idx, w, out, body)
            count += 1
        per_expert = (time.perf_counter() - t0) / count
        layer_s = per_expert * EXPERTS
        return {"value": round(PREFILL_TOKENS / layer_s, 2), "unit": "token-layers/s", "cores": 1, "kind": "port",
                "sample": f"{count} runs of one expert's 64-token share (gate, up, SwiGLU, down selected-token "
                          f"matmuls) in {per_expert * 1e3:.0f} ms each, times 32 experts = one 512-token layer; "
                          f"oracle restatement of tensor.cpp:319-495 / model.cpp:378-460 (the matmul's token loop "
                          f"auto-vectorized, -O3 -ffp-contract=off -march=x86-64-v3)"}
    if workload == "model-prefill":
        from model_fixtures import HostModelLayer

        # one sliding-window and one full layer (4 experts, all selected) of the oracle's
        # layer-major prefill over a 32-token sample; a token costs the mean of the two
        # per layer, times the model's layers
        host_layers = [HostModelLayer(SEED, l, 4) for l in (0, 1)]
        freqs = np.empty(32, np.float32)
        O.lib.orc_rope_frequencies(freqs)
        sample = 32
        x = O.synth_normal(0x78000310, 0, sample * N)
        out = np.empty(sample * N, np.float32)
        kc, vc = np.zeros(sample * 512, np.float32), np.zeros(sample * 512, np.float32)
        runs, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds or runs == 0:
            for l in (0, 1):
                s = host_layers[l].struct()
                O.lib.orc_layer_prefill(C.byref(s), l, 0, sample, x, freqs, kc, vc, body, out, None)
            runs += 1
        per_token_layer = (time.perf_counter() - t0) / (runs * 2 * sample)
        return {"value": round(1.0 / (per_token_layer * layers), 3), "unit": "prompt tok/s", "cores": 1,
                "kind": "port",
                "sample": f"{runs} x (one window + one full layer) of the oracle's prefill (model.cpp:484-553) over "
                          f"{sample} tokens, {per_token_layer * 1e3:.2f} ms per token-layer, times {layers} layers; "
                          f"MXFP4 {isa}, Q8_0 matmuls as the reference's C loops"}

    if workload == "matvec":
        # config 0 on the CPU: the 5760 x 2880 matrix as two 2880-row experts
        # (matvec_add_mxfp4_2880, tensor.cpp:239-304), over 16 copies (141 MB, beyond
        # the host caches)
        copies = 16
        mats = [O.synth_mxfp4(0x77000000, 100 + i, 2 * N * 90) for i in range(copies)]
        x = O.synth_normal(0x78000000, 0, N)
        zero = np.zeros(2 * N, np.float32)
        y = np.empty(N, np.float32)
        count, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds or count == 0:
            m = mats[count % copies]
            O.lib.orc_matvec_add_mxfp4(m, zero, N, N, x, y, 0, body)
            O.lib.orc_matvec_add_mxfp4(m, zero, N, N, x, y, 1, body)
            count += 1
        per = (time.perf_counter() - t0) / count
        return {"value": round(MATVEC_BYTES / per / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{count} config-0 matvecs (two 2880-row experts each) over {copies} distinct matrices, "
                          f"{per * 1e3:.2f} ms each; oracle restatement of tensor.cpp:239-304, {isa}"}
    if workload == "moe":
        from moe_fixtures import HostLayer

        host = HostLayer(EXPERTS, USED, biases=False, seed=0x77000100)
        out = np.empty(N, np.float32)
        s = host.oracle_struct()
        xs = [O.synth_normal(0x78000200, t, N) for t in range(16)]
        count, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            O.lib.orc_moe(C.byref(s), xs[count % 16], out, body, None, None, None)
            count += 1
        elapsed = time.perf_counter() - t0
        return {"value": round(count / elapsed, 3), "unit": "token-layers/s", "cores": 1, "kind": "port",
                "sample": f"{count} token-layers of config 1 in {elapsed:.1f} s; oracle restatement of tensor.cpp "
                          f"matvecs + model.cpp moe; {isa}"}

    from model_fixtures import HostModelLayer

    # Layers with 4 experts (all selected): the same per-token work as 4 of 32.
    host_layers = [HostModelLayer(SEED, l, 4) for l in (0, 1)]
    freqs = np.empty(32, np.float32)
    O.lib.orc_rope_frequencies(freqs)
    cap = context + 1
    kc = O.synth_normal(0x78000300, 1, cap * 512)
    vc = O.synth_normal(0x78000300, 2, cap * 512)
    x = O.synth_normal(0x78000300, 3, N, sigma=30.0)
    outs = {k: np.empty(n, np.float32) for k, n in (("x", N), ("q", 4096), ("a", 4096), ("r", N), ("ro", 4))}
    idx, w = np.empty(4, np.int64), np.empty(4, np.float32)
    times = {0: [], 1: []}
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds * 0.6 or not times[1]:
        for l in (0, 1):
            s = host_layers[l].struct()
            t = time.perf_counter()
            O.lib.orc_layer_forward(C.byref(s), l, context, x, freqs, kc, vc, body, outs["x"], outs["q"], outs["a"],
                                    outs["r"], outs["ro"], idx, w)
            times[l].append(time.perf_counter() - t)
    unembed = O.synth_bf16(SEED, 3 * 1000, VOCAB * N)
    logits = np.empty(VOCAB, np.float32)
    t = time.perf_counter()
    O.lib.orc_matvec_bf16(unembed, VOCAB, N, x, logits)
    t_logits = time.perf_counter() - t
    t_window, t_full = float(np.median(times[0])), float(np.median(times[1]))
    t_token = (layers // 2) * t_window + (layers - layers // 2) * t_full + t_logits
    return {"value": round(1.0 / t_token, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"oracle restatement of model.cpp forward at position {context}: median of {len(times[0])} "
                      f"window-layer ({t_window * 1e3:.0f} ms) and {len(times[1])} full-context-layer "
                      f"({t_full * 1e3:.0f} ms) runs plus one 201088-row bf16 unembedding ({t_logits * 1e3:.0f} ms); "
                      f"token = {layers // 2} + {layers - layers // 2} layers + unembedding; MXFP4 {isa}, other matvecs "
                      f"as the reference's C loops "
                      f"(-O3 -ffp-contract=off -march=x86-64-v3)"}


def _summary(res, kernel_keys=("kernel", "launch_us", "GBps", "achieved", "frac", "bytes_per_launch",
                                 "mfma_algorithmic_TFLOPs", "mfma_peak_TFLOPs")):
    roof = {k: v for k, v in res["roofline"].items() if k in kernel_keys}
    ceiling = res["roofline"].get("read_ceiling")
    if ceiling:
        roof["read_ceiling_us"] = ceiling["launch_us"]
        roof["kernel_frac_of_ceiling"] = ceiling["kernel_frac_of_ceiling"]
    out = {"workload": res["config"]["workload"], "value": round(res["value"], 2), "unit": res["unit"],
           "ms_per_step": round(res["ms_per_step"], 5), "roofline": roof}
    if "dtype" in res:
        out["dtype"] = res["dtype"]
    return out


def other_configs(args):
    """Configs 1, 2 (both arithmetic paths) and 4 in the default run, so that the driver's
    own run measures every BASELINE config: each is its own workload's measurement
    (--workload moe / prefill / decode --config 4) with fewer steps, summarized."""
    import copy

    out = {}
    a = copy.copy(args)
    a.steps, a.warmup = 40, 5
    t0 = time.time()
    out["config1"] = _summary(gpu_moe(a))
    log(f"config 1: {out['config1']['value']:.0f} token-layers/s ({time.time() - t0:.1f} s)")
    for act in ("bf16", "mxfp8"):
        t0 = time.time()
        a = copy.copy(args)
        a.steps, a.warmup, a.activations = 60, 3, act
        out[f"config2_{act}"] = _summary(gpu_prefill(a))
        log(f"config 2 ({act}): {out[f'config2_{act}']['value']:.0f} token-layers/s ({time.time() - t0:.1f} s)")
    t0 = time.time()
    a = copy.copy(args)
    a.config, a.experts, a.layers, a.context = 4, 128, 36, 4096
    a.steps, a.warmup, a.table, a.skip_matvec = 20, 5, None, True
    out["config4"] = _summary(gpu_decode(a))
    log(f"config 4: {out['config4']['value']:.1f} tok/s ({time.time() - t0:.1f} s)")
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=["decode", "matvec", "moe", "prefill", "model-prefill"], default="decode")
    ap.add_argument("--activations", choices=["bf16", "mxfp8"], default="bf16",
                    help="prefill workload: bf16 MFMA on bf16 activations (exact), or the scaled path "
                         "(activations and hidden quantized to MXFP8, fp8 x fp4 MFMA)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="launch each step's kernels one by one instead of replaying the step graph "
                         "(for kernel tracers that cannot follow graph launches)")
    ap.add_argument("--config", type=int, choices=[3, 4], default=3,
                    help="decode workload: 3 = gpt-oss-20b shape (24 layers, 32 experts, KV 2048; the headline), "
                         "4 = gpt-oss-120b shape (36 layers, 128 experts, KV 4096)")
    ap.add_argument("--context", type=int, default=None,
                    help="KV positions filled before timing (default: 2048 for config 3, 4096 for config 4)")
    ap.add_argument("--layers", type=int, default=None,
                    help="decoder layers (default 24 / 36; fewer only for counter probes)")
    ap.add_argument("--kv-fill", choices=["decode", "synthetic"], default="decode",
                    help="decode workload: fill the KV caches by decoding (the benchmark) or with synthetic "
                         "values (counter runs, whose profilers serialize every launch)")
    ap.add_argument("--table", default=None,
                    help="decode workload: also write the per-kind kernel table (text) to this path")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="decode workload: skip configs 1, 2 and 4, which the default run also measures "
                         "(the line's other_configs field)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first copy this many MiB device-to-device once, a known-size reference "
                         "dispatch for scaling hardware byte counters")
    args = ap.parse_args()
    args.experts = EXPERTS if args.config == 3 else 128
    if args.layers is None:
        args.layers = LAYERS if args.config == 3 else 36
    if args.context is None:
        args.context = CONTEXT if args.config == 3 else 4096
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe_mib:
        import ttlab_amd

        dev = ttlab_amd.Device(0)
        n = args.copy_probe_mib << 20
        src, dst = dev.alloc(n), dev.alloc(n)
        dev.fill(src, 1)
        dev.sync()
        dev.copy(dst, src, n)
        dev.sync()
        log(f"copy probe: {n} bytes device to device")
        src.free()
        dst.free()
        dev.close()
    runner = {"decode": gpu_decode, "matvec": gpu_matvec, "moe": gpu_moe, "prefill": gpu_prefill,
              "model-prefill": gpu_model_prefill}[args.workload]
    res = runner(args)
    base = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds, args.workload, args.layers, args.context)
    if base:
        log(f"cpu baseline: {base['value']} {base['unit']}")
    line = {
        "metric": METRIC,
        "value": round(res["value"], 2),
        "unit": res["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res.get("dtype", "f32 (MXFP4/Q8_0/bf16 weights)"),
        "data": "synthetic",
        "config": dict(res["config"], launch="eager" if args.eager else "hip graph"),
        "roofline": res["roofline"],
        "cpu_baseline": base,
    }
    if res.get("matvec"):
        line["matvec"] = res["matvec"]
    if args.workload == "decode" and args.config == 3 and not args.no_other_configs:
        line["other_configs"] = other_configs(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
