"""Benchmark of the quantized MoE expert path on one MI355X.

Headline workload (the metric's decode target): the
Kimi-K2 MoE layer on one GPU's 48 local experts, 64 decode tokens, sigmoid
top-8 routing from seeded N(0,1) logits -- router select, permutation,
W13 grouped GEMM, SwiGLU, W2 grouped GEMM with routing weights, top-k combine.
One step = one layer over resident inputs.  `value` is the layer's achieved
HBM bandwidth over its algorithmic bytes (touched experts' weights + scales,
activations in, routed output); the roofline block reports the dominant
kernel (the W13 GEMM) timed with HIP events on its own stream inside the
timed steps.  The other configurations (C1, C2, C4, C5) are reported under
"configs"; the CPU baseline times the oracle's C restatement of the same
layer on the host's cores.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only c3]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("MoE layer µs + achieved HBM GB/s (decode) / MFMA TFLOP/s (prefill) on 1 MI355X")
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
W13_BYTES_PER_EXPERT = 4096 * 7168 // 2 + 4096 * (7168 // 32) * 2  # 16,515,072
W2_BYTES_PER_EXPERT = 7168 * 2048 // 2 + 7168 * (2048 // 32) * 2  # 8,257,536


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--only", default="", help="comma list of configs to run (c1..c5)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a plain 256 MiB device copy (reference kernel for the "
                        "FETCH_SIZE / WRITE_SIZE counter scale) and exit")
    p.add_argument("--clock-ramp", action="store_true",
                   help="only time the C3 graph in consecutive passes from a cold start "
                        "(the evidence for WARM_MS) and exit")
    return p.parse_args()


def calibrate_copy(torch):
    n = 256 * 1024 * 1024 // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": n * 4, "bytes_written": n * 4,
                      "launches": 5}))


def clock_ramp(torch):
    """The C3 four-layer graph timed in consecutive passes of 20 replays: from 5 warm-up
    replays, then again after 2 s idle.  The per-layer mean of each pass shows how long
    the GPU takes to reach its steady clock (the reason for WARM_MS)."""
    import numpy as np
    from pegainfer_amd import layer, ops, synth
    E, H, I, T = 48, 7168, 2048, 64
    g = synth.rng(3, 1)
    gate, up, down = (synth.int4_checkpoint(g, E, I, H), synth.int4_checkpoint(g, E, I, H),
                      synth.int4_checkpoint(g, E, H, I))
    hidden = dev(torch, synth.normal_bf16(synth.rng(3, 2), (T, H)), bf16=True)
    logits = dev(torch, synth.rng(3, 3).standard_normal((T, 384), dtype=np.float32))
    bias = torch.zeros(384, dtype=torch.float32, device="cuda")
    tw = torch.zeros(T, 8, dtype=torch.float32, device="cuda")
    ti = torch.zeros(T, 8, dtype=torch.int32, device="cuda")
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    layers = [layer.RoutedExperts(layer.package_w13(gate, up), layer.package_projection(*down),
                                  max_tokens=T, topk=8, block_size=ops.kimi_marlin_block_size(T))
              for _ in range(GRAPH_LAYERS)]

    def step_layers():
        for m in layers:
            m.forward_from_logits(hidden, logits, bias, tw, ti, out)
    graph = layer.capture_graph(step_layers)

    def passes(n, steps=20):
        res = []
        for _ in range(n):
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(torch.cuda.current_stream())
            for _ in range(steps):
                graph.replay()
            e1.record(torch.cuda.current_stream())
            torch.cuda.synchronize()
            res.append(round(e0.elapsed_time(e1) * 1e3 / (steps * GRAPH_LAYERS), 1))
        return res
    for _ in range(5):
        graph.replay()
    cold = passes(12)
    time.sleep(2.0)
    idle = passes(6)
    print(json.dumps({"clock_ramp": "c3 graph, per-layer us per pass of 20 replays "
                                    "(4 layers each, about 15 ms)",
                      "after_5_warmup_replays": cold, "after_2s_idle": idle}))


class EventTimer:
    """Pairs of HIP events recorded on the stream the kernels run on."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []

    def start(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.torch.cuda.current_stream())
        return e

    def stop(self, s):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.torch.cuda.current_stream())
        self.pairs.append((s, e))

    def mean_ms(self):
        self.torch.cuda.synchronize()
        if not self.pairs:
            return float("nan")
        return sum(s.elapsed_time(e) for s, e in self.pairs) / len(self.pairs)


# An MI355X coming out of idle ramps its clocks over its first ~20 ms of load (the C3
# graph: 204 us per layer over the first 20 replays after 5 warm-ups, 181 us from then
# on, and 213 us again after 2 s idle), so every warm-up below also runs until the GPU
# has been busy for WARM_MS: a short warm-up would leave part of the ramp in the timed
# window.  The timed steps themselves are unchanged.
WARM_MS = 50.0


def warm(torch, fn, count):
    """`count` untimed calls of `fn`, then more, one at a time, until WARM_MS of wall
    time has passed since the first."""
    t0 = time.perf_counter()
    n = 0
    while n < count or (time.perf_counter() - t0) * 1e3 < WARM_MS:
        fn()
        n += 1
        if n >= count:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def time_steps(torch, fn, steps, warmup):
    warm(torch, fn, warmup)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


GRAPH_CALLS = 16  # consecutive small-batch forwards per captured graph
# C3 headline: decode layers per captured graph, each with its own copy of the
# 48 experts' packed weights (distinct buffers, so no layer's weights are
# cache-resident for the next: 4 layers stream ~3.7 GB against a 256 MB MALL),
# as a decode step replays every layer of the model in one graph.
GRAPH_LAYERS = 4
# copies of the shared expert's weights the kernel-alone figures rotate through
SHARED_COPIES = 4


def time_graph(torch, fn, steps, warmup, calls=GRAPH_CALLS):
    """Per-call time of `fn` captured `calls` times back to back into one HIP
    graph (as a decode step replays many layers), timed with events around
    `steps` replays.  Host launch overhead, which dominates a few-microsecond
    eager launch from Python, is out of the measurement; every call still does
    its full work."""
    from pegainfer_amd import layer
    graph = layer.capture_graph(lambda: [fn() for _ in range(calls)])
    warm(torch, graph.replay, warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(torch.cuda.current_stream())
    for _ in range(steps):
        graph.replay()
    e1.record(torch.cuda.current_stream())
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (steps * calls)


def attainable_read(torch, nbytes):
    """The GPU's attainable HBM read rate, measured here: a plain streaming-read kernel
    (pegainfer_amd/libpega_hbm_probe.so, measurement only) over `nbytes` per launch,
    rotating through four buffers (more than the 256 MB MALL holds), 16 launches per
    HIP graph; the best of three grid sizes.  Reported beside the roofline fraction as
    what a kernel with no compute reaches on the same box."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "pegainfer_amd", "libpega_hbm_probe.so"))
    fn = lib.pega_hbm_read_probe
    fn.argtypes = [ctypes.c_void_p, ctypes.c_ulonglong, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p]
    nbytes -= nbytes % 16
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device="cuda") for _ in range(4)]
    best = None
    for grid in (512, 1024, 2048):
        out = torch.empty(grid * 256, dtype=torch.int32, device="cuda")
        turn = [0]

        def launch():
            b = bufs[turn[0] % 4]
            turn[0] += 1
            rc = fn(b.data_ptr(), nbytes, out.data_ptr(), grid,
                    torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError("pega_hbm_read_probe failed")
        ms = time_graph(torch, launch, 5, 2)
        gbs = nbytes / (ms * 1e-3) / 1e9
        if best is None or gbs > best["value"]:
            best = dict(value=round(gbs, 1), unit="GB/s", grid=grid, launch_us=round(ms * 1e3, 2))
    del bufs
    torch.cuda.empty_cache()
    best.update(kernel="hbm_read_kernel (contiguous chunk per workgroup, 16-byte "
                       "non-temporal loads, 4 in flight per thread)", bytes_per_launch=nbytes)
    return best


def dev(torch, a, bf16=False):
    import numpy as np
    a = np.ascontiguousarray(a)
    if bf16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


# ----------------------------------------------------------------------------- C3
def bench_c3(torch, args, results):
    import numpy as np
    from pegainfer_amd import layer, ops, synth
    E, H, I, T = 48, 7168, 2048, 64
    log("C3: generating 48 experts (seeded) and packing on the GPU")
    g = synth.rng(3, 1)
    gate, up, down = (synth.int4_checkpoint(g, E, I, H), synth.int4_checkpoint(g, E, I, H),
                      synth.int4_checkpoint(g, E, H, I))
    hidden_np = synth.normal_bf16(synth.rng(3, 2), (T, H))
    logits_np = synth.rng(3, 3).standard_normal((T, 384), dtype=np.float32)
    bs = ops.kimi_marlin_block_size(T)
    moe = layer.RoutedExperts(layer.package_w13(gate, up), layer.package_projection(*down),
                              max_tokens=T, topk=8, block_size=bs)
    hidden = dev(torch, hidden_np, bf16=True)
    logits = dev(torch, logits_np)
    bias = torch.zeros(384, dtype=torch.float32, device="cuda")
    tw = torch.zeros(T, 8, dtype=torch.float32, device="cuda")
    ti = torch.zeros(T, 8, dtype=torch.int32, device="cuda")
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    timer = EventTimer(torch)

    def step(record=False):
        moe.forward_from_logits(hidden, logits, bias, tw, ti, out,
                                w13_timer=timer if record else None)

    step()
    torch.cuda.synchronize()
    idx = ti.cpu().numpy()
    touched = np.unique(idx[idx < E]).size
    local_routes = int((idx < E).sum())
    alg_bytes = (touched * (W13_BYTES_PER_EXPERT + W2_BYTES_PER_EXPERT) + T * H * 2 + T * H * 4)
    # W13 + SwiGLU: weights and scales of the touched experts, the tokens' activations
    # in, the routed rows' SwiGLU activations out
    w13_bytes = touched * W13_BYTES_PER_EXPERT + T * H * 2 + local_routes * I * 2
    log(f"C3: block size {bs}, {touched} experts touched, {local_routes} local routes, "
        f"{alg_bytes / 1e6:.1f} MB algorithmic")
    # Eager launches, W13 timed with events on its stream (the roofline kernel).
    warm(torch, step, args.warmup)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(record=True)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    w13_ms = timer.mean_ms()
    # The headline: GRAPH_LAYERS decode layers (router select + routed experts
    # each, every layer on its own copy of the packed weights) captured into one
    # HIP graph and replayed, as a decode step runs the model's layers; the
    # figure is per layer.  One layer per graph is reported beside it: there
    # each replay also pays the graph launch.
    layers = [moe] + [
        layer.RoutedExperts(layer.package_w13(gate, up), layer.package_projection(*down),
                            max_tokens=T, topk=8, block_size=bs)
        for _ in range(GRAPH_LAYERS - 1)]

    def replay_ms(graph, n):
        warm(torch, graph.replay, args.warmup)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(torch.cuda.current_stream())
        for _ in range(args.steps):
            graph.replay()
        e1.record(torch.cuda.current_stream())
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (args.steps * n)

    def replay_spread_us(graph, n, count=100):
        """Median and p99 of the per-layer time over `count` replays, each between
        its own pair of events (the mean above has no per-replay event in the way)."""
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(count + 1)]
        ev[0].record(torch.cuda.current_stream())
        for i in range(count):
            graph.replay()
            ev[i + 1].record(torch.cuda.current_stream())
        torch.cuda.synchronize()
        per = sorted(ev[i].elapsed_time(ev[i + 1]) * 1e3 / n for i in range(count))
        return per[count // 2], per[min(count - 1, (99 * count + 99) // 100 - 1)]

    def step_layers():
        for m in layers:
            m.forward_from_logits(hidden, logits, bias, tw, ti, out)
    layers_graph = layer.capture_graph(step_layers)
    ms = replay_ms(layers_graph, GRAPH_LAYERS)
    med_us, p99_us = replay_spread_us(layers_graph, GRAPH_LAYERS)
    del layers_graph
    ms_one = replay_ms(layer.capture_graph(step), 1)
    del layers[1:]
    # The roofline kernel alone: the W13 + SwiGLU launch with the layer's routing,
    # captured GRAPH_CALLS times back to back and replayed, so the figure is the
    # kernel's own duration (no host launch gaps), the quantity a kernel trace reports.
    routing = moe.routing
    act = moe.act[:T * 8]
    w13_graph_ms = time_graph(
        torch, lambda: ops.wna16_w13_swiglu(moe.gemm_ws, routing, hidden, moe.w13, act, top_k=8,
                                            size_m=T), args.steps, args.warmup)
    w2_graph_ms = time_graph(
        torch, lambda: ops.wna16_gemm(moe.gemm_ws, routing, act, moe.w2, tw, moe.route_out[:T * 8],
                                      top_k=1, mul_topk_weights=True, size_m=T * 8),
        args.steps, args.warmup)
    w2_bytes = touched * W2_BYTES_PER_EXPERT + local_routes * I * 2 + local_routes * H * 2
    # The layer's routing alone: the fused select + permutation launch it uses, and the
    # select and permutation launches it replaces (same outputs, bit for bit).
    route_fused_ms = time_graph(
        torch, lambda: ops.kimi_route_align(moe.route_ws, logits, bias, tw, ti, T, 0),
        args.steps, args.warmup)

    def two_launches():
        ops.kimi_router_select(logits, bias, tw, ti, T)
        ops.moe_align_block_size(moe.route_ws, ti, T, T, 0)
    route_two_ms = time_graph(torch, two_launches, args.steps, args.warmup)
    results["c3"] = dict(
        workload="c3_kimi_moe_decode_t64", tokens=T, local_experts=E, hidden=H, inter=I, topk=8,
        block_size=bs, touched_experts=touched, local_routes=local_routes,
        algorithmic_bytes=alg_bytes, layer_us=ms * 1e3, layer_us_eager=eager_ms * 1e3,
        graph_layers=GRAPH_LAYERS, layer_us_median=med_us, layer_us_p99=p99_us,
        layer_us_one_per_graph=ms_one * 1e3,
        layer_gbs=alg_bytes / (ms * 1e-3) / 1e9, w13_us=w13_graph_ms * 1e3,
        w13_us_in_eager_layer=w13_ms * 1e3,
        w13_algorithmic_bytes=w13_bytes, w13_gbs=w13_bytes / (w13_graph_ms * 1e-3) / 1e9,
        w2_us=w2_graph_ms * 1e3, w2_algorithmic_bytes=w2_bytes,
        w2_gbs=w2_bytes / (w2_graph_ms * 1e-3) / 1e9,
        route_fused_us=route_fused_ms * 1e3, route_two_launches_us=route_two_ms * 1e3)
    log(f"C3: layer {ms * 1e3:.1f} us graph-replayed ({GRAPH_LAYERS} layers per graph, "
        f"{results['c3']['layer_gbs']:.0f} GB/s), {ms_one * 1e3:.1f} us one layer per graph, "
        f"{eager_ms * 1e3:.1f} us eager; W13+SwiGLU {w13_graph_ms * 1e3:.1f} us alone "
        f"({results['c3']['w13_gbs']:.0f} GB/s; {w13_ms * 1e3:.1f} us in the eager layer), "
        f"W2 {w2_graph_ms * 1e3:.1f} us alone ({results['c3']['w2_gbs']:.0f} GB/s); routing "
        f"{route_fused_ms * 1e3:.1f} us fused, {route_two_ms * 1e3:.1f} us as two launches")
    bench_c3_shared(torch, args, results, moe, hidden, logits, bias)
    return dict(gate=gate, up=up, down=down, hidden=hidden_np, idx=idx,
                w=tw.cpu().numpy(), bs=bs, alg_bytes=alg_bytes)


def host_threads():
    """Host cores this process may use: the CPUs it is pinned to, at most 16 (a GPU
    box gives one GPU's job 16 host cores, whatever the machine has in total)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline_c3(ctx, results):
    """The CPU restatement of the same C3 layer (oracle/moe_oracle.c: the vectorised
    GEMM variant, pthreads over (m-block, 64-column) work items, SwiGLU, fp32 top-k
    sum) on the host's cores: median of 5 layers on every allowed core, and of 3 on
    one core."""
    import statistics
    import numpy as np
    from oracle import oracle
    threads = host_threads()
    w13p = np.concatenate([ctx["gate"][0], ctx["up"][0]], axis=1)
    w13s = np.concatenate([ctx["gate"][1], ctx["up"][1]], axis=1)

    def layer_s(nthreads):
        t0 = time.perf_counter()
        oracle.kimi_moe_layer(ctx["hidden"], w13p, w13s, ctx["down"][0], ctx["down"][1],
                              ctx["idx"].reshape(-1), ctx["w"], global_start=0, local_experts=48,
                              block_size=ctx["bs"], hidden=7168, inter=2048, threads=nthreads,
                              fast=True)
        return time.perf_counter() - t0
    layer_s(threads)  # first touch of the weights
    multi = statistics.median(layer_s(threads) for _ in range(5))
    single = statistics.median(layer_s(1) for _ in range(3))
    results["cpu"] = dict(value=ctx["alg_bytes"] / multi / 1e9, unit="GB/s", cores=threads,
                          kind="port",
                          sample=f"median of 5 full C3 layers (64 tokens, 48 experts, "
                                 f"{ctx['alg_bytes'] / 1e6:.0f} MB) on {threads} threads; "
                                 f"1-thread median of 3",
                          layer_ms=multi * 1e3, layer_ms_1thread=single * 1e3,
                          value_1thread=ctx["alg_bytes"] / single / 1e9)
    log(f"CPU baseline: {multi * 1e3:.0f} ms per layer on {threads} threads, "
        f"{single * 1e3:.0f} ms on 1")


def bench_c3_shared(torch, args, results, moe, normed, logits, bias):
    """Beside the C3 routed layer: the Kimi shared expert (bf16 dense MLP, gate/up
    [4096, 7168] and down [7168, 2048], seeded N(0, 0.02) weights) on the same 64
    tokens, its gate/up GEMM with the SwiGLU epilogue alone, and the whole decode layer (shared expert,
    router select, routed experts, residual join) as one HIP graph."""
    import numpy as np
    from pegainfer_amd import layer, synth
    T, H, SI = 64, 7168, 2048
    g = synth.rng(3, 4)
    gu = dev(torch, synth.normal_bf16(g, (2 * SI, H), std=0.02), bf16=True)
    dn = dev(torch, synth.normal_bf16(g, (H, SI), std=0.02), bf16=True)
    shared = layer.KimiSharedExpert(gu, dn, max_tokens=T)
    full = layer.KimiMoeDecodeLayer(moe, shared)
    hidden = dev(torch, synth.normal_bf16(synth.rng(3, 5), (T, H)), bf16=True)
    proj = torch.zeros(T, H, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(T, H, dtype=torch.bfloat16, device="cuda")
    from pegainfer_amd import ops
    # The kernel-alone figures rotate through SHARED_COPIES copies of the weights
    # (88 MB each, more than the 256 MB MALL together), so every call streams its
    # weights from HBM rather than from the previous call's cache.
    copies = [shared] + [layer.KimiSharedExpert(gu.clone(), dn.clone(), max_tokens=T)
                         for _ in range(SHARED_COPIES - 1)]
    gemm_ms = time_graph(
        torch, lambda: [ops.dense_w13_swiglu(m.gate_up, normed, m.act[:T]) for m in copies],
        args.steps, args.warmup) / SHARED_COPIES
    shared_ms = time_graph(torch, lambda: [m.forward(normed, proj) for m in copies], args.steps,
                           args.warmup) / SHARED_COPIES
    del copies[1:]
    graph = layer.capture_graph(lambda: full.forward(hidden, normed, logits, bias, out))
    warm(torch, graph.replay, args.warmup)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(torch.cuda.current_stream())
    for _ in range(args.steps):
        graph.replay()
    e1.record(torch.cuda.current_stream())
    torch.cuda.synchronize()
    full_ms = e0.elapsed_time(e1) / args.steps
    gemm_bytes = 2 * SI * H * 2 + T * H * 2 + T * SI * 2
    # weights, the input and output rows, and the SwiGLU activations written by
    # the gate/up launch and read back by the down GEMM
    shared_bytes = (2 * SI * H + H * SI) * 2 + T * H * 2 * 2 + 2 * T * SI * 2
    results["c3_shared"] = dict(
        workload="c3_kimi_shared_expert_t64", tokens=T, hidden=H, inter=SI,
        launch=f"hip_graph ({GRAPH_CALLS} calls per graph over {SHARED_COPIES} weight copies)",
        gate_up_us=gemm_ms * 1e3, gate_up_bytes=gemm_bytes,
        gate_up_gbs=gemm_bytes / (gemm_ms * 1e-3) / 1e9,
        shared_us=shared_ms * 1e3, shared_bytes=shared_bytes,
        shared_gbs=shared_bytes / (shared_ms * 1e-3) / 1e9,
        full_layer_us=full_ms * 1e3)
    log(f"C3 shared expert: gate/up GEMM + SwiGLU {gemm_ms * 1e3:.1f} us "
        f"({results['c3_shared']['gate_up_gbs']:.0f} GB/s), shared MLP {shared_ms * 1e3:.1f} us "
        f"({results['c3_shared']['shared_gbs']:.0f} GB/s); full decode layer (shared + routed + "
        f"join) {full_ms * 1e3:.1f} us graph-replayed")


# ----------------------------------------------------------------------------- C1/C2
def bench_c1(torch, args, results):
    from pegainfer_amd import layer, synth
    g = synth.rng(1, 1)
    packed, scales = synth.int4_checkpoint(g, 1, 9728, 2560)
    dense = layer.DenseW4A16(layer.package_projection(packed, scales), max_rows=1)
    x = dev(torch, synth.normal_bf16(synth.rng(1, 2), (1, 2560)), bf16=True)
    y = torch.zeros(1, 9728, dtype=torch.bfloat16, device="cuda")
    eager_ms = time_steps(torch, lambda: dense.forward(x, y), max(args.steps, 200), args.warmup)
    ms = time_graph(torch, lambda: dense.forward(x, y), max(args.steps // 4, 50), args.warmup)
    b = 14_032_896
    results["c1"] = dict(workload="c1_dense_gemv_9728x2560", us=ms * 1e3, us_eager=eager_ms * 1e3,
                         launch=f"hip_graph ({GRAPH_CALLS} calls per graph)",
                         gbs=b / (ms * 1e-3) / 1e9, algorithmic_bytes=b)
    log(f"C1: {ms * 1e3:.2f} us graph-replayed ({results['c1']['gbs']:.0f} GB/s), "
        f"{eager_ms * 1e3:.2f} us eager")
    if not args.no_cpu:
        cpu_c1(results["c1"], packed, scales, synth.normal_bf16(synth.rng(1, 2), (1, 2560)))


def cpu_c1(res, packed, scales, x_bits):
    """C1 is the reference's CPU-runnable case: the oracle GEMV on the same
    inputs, on 1 thread (best of 5 runs) and on up to 16 (best of 20)."""
    import numpy as np
    from oracle import oracle
    routing = dict(sorted_token_ids=np.array([0] + [1] * 7, np.int32),
                   expert_ids=np.zeros(1, np.int32),
                   num_tokens_post_padded=np.array([8], np.int32))
    kw = dict(moe_block_size=8, top_k=1, mul_topk_weights=False, size_m=1, size_n=9728,
              size_k=2560)
    for threads in sorted({1, host_threads()}):
        best = float("inf")
        for _ in range(5 if threads == 1 else 20):
            t0 = time.perf_counter()
            oracle.wna16_gemm(x_bits, packed, scales, routing, np.ones(1, np.float32),
                              threads=threads, **kw)
            best = min(best, time.perf_counter() - t0)
        res[f"cpu_us_{threads}t"] = best * 1e6
    res["cpu_kind"] = "port"
    log("C1 CPU (oracle): " + ", ".join(f"{v:.0f} us on {k[7:-1]} thread(s)"
                                         for k, v in res.items() if k.startswith("cpu_us_")))


def bench_c2(torch, args, results):
    from pegainfer_amd import layer, synth
    g = synth.rng(2, 1)
    gate, up, down = (synth.int4_checkpoint(g, 1, 2048, 7168), synth.int4_checkpoint(g, 1, 2048, 7168),
                      synth.int4_checkpoint(g, 1, 7168, 2048))
    ffn = layer.ExpertFFN(layer.package_w13(gate, up), layer.package_projection(*down), max_rows=8)
    out = {}
    for b in (1, 4, 8):
        x = dev(torch, synth.normal_bf16(synth.rng(2, 2), (b, 7168)), bf16=True)
        y = torch.zeros(b, 7168, dtype=torch.bfloat16, device="cuda")
        eager_ms = time_steps(torch, lambda: ffn.forward(x, y), max(args.steps, 200), args.warmup)
        ms = time_graph(torch, lambda: ffn.forward(x, y), max(args.steps // 4, 50), args.warmup)
        nbytes = W13_BYTES_PER_EXPERT + W2_BYTES_PER_EXPERT + b * 7168 * 4
        out[f"b{b}"] = dict(us=ms * 1e3, us_eager=eager_ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9)
        log(f"C2 b={b}: {ms * 1e3:.2f} us graph-replayed ({out[f'b{b}']['gbs']:.0f} GB/s), "
            f"{eager_ms * 1e3:.2f} us eager")
    results["c2"] = dict(workload="c2_kimi_expert_ffn",
                         launch=f"hip_graph ({GRAPH_CALLS} calls per graph)", **out)


# ----------------------------------------------------------------------------- C4/C5
def bench_c4(torch, args, results):
    import numpy as np
    from pegainfer_amd import layer, ops, synth
    E, H, I, T, topk = 64, 2048, 1408, 512, 6
    g = synth.rng(4, 1)
    gate, up, down = (synth.int4_checkpoint(g, E, I, H), synth.int4_checkpoint(g, E, I, H),
                      synth.int4_checkpoint(g, E, H, I))
    sg, su, sd = (synth.int4_checkpoint(g, 1, 2 * I, H), synth.int4_checkpoint(g, 1, 2 * I, H),
                  synth.int4_checkpoint(g, 1, H, 2 * I))
    bs = ops.kimi_marlin_block_size(T, topk=topk, local_experts=E)
    routed = layer.RoutedExperts(layer.package_w13(gate, up), layer.package_projection(*down),
                                 max_tokens=T, topk=topk, block_size=bs)
    shared = layer.ExpertFFN(layer.package_w13(sg, su), layer.package_projection(*sd), max_rows=T)
    moe = layer.Dsv2MoeLayer(routed, shared)
    hidden = dev(torch, synth.normal_bf16(synth.rng(4, 2), (T, H)), bf16=True)
    logits = dev(torch, synth.rng(4, 3).standard_normal((T, E), dtype=np.float32))
    out = torch.zeros(T, H, dtype=torch.bfloat16, device="cuda")
    eager_ms = time_steps(torch, lambda: moe.forward(hidden, logits, out), args.steps,
                          args.warmup)
    ms = time_graph(torch, lambda: moe.forward(hidden, logits, out), args.steps, args.warmup,
                    calls=1)
    flops = 2 * T * topk * (2 * I * H + H * I) + 2 * T * (2 * 2 * I * H + H * 2 * I)
    results["c4"] = dict(workload="c4_dsv2lite_moe_prefill_t512", us=ms * 1e3,
                         us_eager=eager_ms * 1e3, launch="hip_graph",
                         tflops=flops / (ms * 1e-3) / 1e12, flops=flops, block_size=bs)
    log(f"C4: {ms * 1e3:.1f} us graph-replayed ({results['c4']['tflops']:.1f} TFLOP/s), "
        f"{eager_ms * 1e3:.1f} us eager")


def bench_c5(torch, args, results):
    from pegainfer_amd import layer, ops, synth
    E, H, I, T = 48, 7168, 2048, 4096
    g = synth.rng(5, 1)
    gate, up, down = (synth.int4_checkpoint(g, E, I, H), synth.int4_checkpoint(g, E, I, H),
                      synth.int4_checkpoint(g, E, H, I))
    idx, w = synth.zipf_local_topk(synth.rng(5, 3), T)
    routes = int((idx < E).sum())
    bs = ops.kimi_marlin_block_size(T)
    moe = layer.RoutedExperts(layer.package_w13(gate, up), layer.package_projection(*down),
                              max_tokens=T, topk=8, block_size=bs)
    hidden = dev(torch, synth.normal_bf16(synth.rng(5, 2), (T, H)), bf16=True)
    ti, tw = dev(torch, idx), dev(torch, w)
    out = torch.zeros(T, H, dtype=torch.float32, device="cuda")
    steps = max(5, args.steps // 5)
    ms = time_graph(torch, lambda: moe.forward(hidden, ti, tw, out), steps, 2, calls=1)
    routing = moe.routing
    act = moe.act[:T * 8]
    w13_ms = time_graph(torch, lambda: ops.wna16_w13_swiglu(moe.gemm_ws, routing, hidden, moe.w13,
                                                            act, top_k=8, size_m=T),
                        steps, 2, calls=4)
    w2_ms = time_graph(torch, lambda: ops.wna16_gemm(moe.gemm_ws, routing, act, moe.w2, tw,
                                                     moe.route_out[:T * 8], top_k=1,
                                                     mul_topk_weights=True, size_m=T * 8),
                       steps, 2, calls=4)
    flops = 2 * routes * (2 * I * H + H * I)
    w13_flops = 2 * routes * 2 * I * H
    w2_flops = 2 * routes * H * I
    results["c5"] = dict(workload="c5_kimi_prefill_t4096_zipf", routes=routes, us=ms * 1e3,
                         launch="hip_graph", tflops=flops / (ms * 1e-3) / 1e12, flops=flops,
                         w13_us=w13_ms * 1e3, w13_flops=w13_flops,
                         w13_tflops=w13_flops / (w13_ms * 1e-3) / 1e12,
                         w2_us=w2_ms * 1e3, w2_flops=w2_flops,
                         w2_tflops=w2_flops / (w2_ms * 1e-3) / 1e12)
    log(f"C5: R={routes}, layer {ms * 1e3:.1f} us ({results['c5']['tflops']:.1f} TFLOP/s), "
        f"W13+SwiGLU {w13_ms * 1e3:.1f} us ({results['c5']['w13_tflops']:.1f} TFLOP/s), "
        f"W2 {w2_ms * 1e3:.1f} us ({results['c5']['w2_tflops']:.1f} TFLOP/s)")
    del moe
    bench_c5_shared(torch, args, results, hidden)


def bench_c5_shared(torch, args, results, normed):
    """The Kimi shared expert (bf16 dense MLP, gate/up [4096, 7168], down [7168, 2048],
    seeded N(0, 0.02) weights) on C5's 4096 prefill tokens: gate/up GEMM, SwiGLU, down
    GEMM (the reference's prefill sequence, hipBLASLt GEMMs), against bf16 MFMA peak."""
    from pegainfer_amd import layer, ops, synth
    T, H, SI = normed.shape[0], 7168, 2048
    g = synth.rng(5, 4)
    gu = dev(torch, synth.normal_bf16(g, (2 * SI, H), std=0.02), bf16=True)
    dn = dev(torch, synth.normal_bf16(g, (H, SI), std=0.02), bf16=True)
    shared = layer.KimiSharedExpert(gu, dn, max_tokens=T)
    proj = torch.zeros(T, H, dtype=torch.bfloat16, device="cuda")
    steps = max(5, args.steps // 5)
    ms = time_graph(torch, lambda: shared.forward(normed, proj), steps, 2, calls=4)
    gu_ms = time_graph(torch, lambda: ops.gemm_graphsafe(gu, normed, shared.h13[:T]), steps, 2,
                       calls=4)
    flops = 2 * T * (2 * SI * H + H * SI)
    gu_flops = 2 * T * 2 * SI * H
    results["c5_shared"] = dict(
        workload="c5_kimi_shared_expert_t4096", tokens=T, hidden=H, inter=SI,
        launch="hip_graph (4 calls per graph)", us=ms * 1e3, flops=flops,
        tflops=flops / (ms * 1e-3) / 1e12, frac_of_bf16_peak=flops / (ms * 1e-3) / 2.5e15,
        gate_up_us=gu_ms * 1e3, gate_up_tflops=gu_flops / (gu_ms * 1e-3) / 1e12)
    log(f"C5 shared expert (T={T}): MLP {ms * 1e3:.1f} us ({results['c5_shared']['tflops']:.0f} "
        f"TFLOP/s, {results['c5_shared']['frac_of_bf16_peak']:.3f} of bf16 peak), gate/up GEMM "
        f"{gu_ms * 1e3:.1f} us ({results['c5_shared']['gate_up_tflops']:.0f} TFLOP/s)")


def load_traffic(name):
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only (no multi-GPU path); "
                                   "run with --gpus 1"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(2)
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    import pegainfer_amd
    pegainfer_amd.load()
    if args.clock_ramp:
        clock_ramp(torch)
        return
    only = set(x.strip() for x in args.only.split(",") if x.strip())
    want = lambda c: not only or c in only  # noqa: E731
    results = {}
    ctx = bench_c3(torch, args, results)
    # right after C3, in the same clock and thermal state as its W13 timing
    reach = attainable_read(torch, results["c3"]["w13_algorithmic_bytes"])
    log(f"attainable HBM read (plain streaming kernel): {reach['value']:.0f} GB/s")
    for name, fn in (("c1", bench_c1), ("c2", bench_c2), ("c4", bench_c4), ("c5", bench_c5)):
        if want(name):
            fn(torch, args, results)
    if not args.no_cpu:
        cpu_baseline_c3(ctx, results)
    c3 = results["c3"]
    roof = dict(bound="hbm", kernel="wna16_decode16_kernel (W13 with SwiGLU epilogue, C3)",
                achieved=round(c3["w13_gbs"], 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(c3["w13_gbs"] / HBM_PEAK_GBS, 4),
                attainable_read=reach,
                frac_of_attainable=round(c3["w13_gbs"] / reach["value"], 4),
                layer_frac_of_attainable=round(c3["layer_gbs"] / reach["value"], 4),
                traffic=load_traffic("wna16_w13_c3"),
                algorithmic_bytes_per_launch=c3["w13_algorithmic_bytes"],
                launch_us=round(c3["w13_us"], 2),
                timing=f"HIP events around graph replays of {GRAPH_CALLS} back-to-back "
                       "launches of this kernel alone (the kernel trace's average of the "
                       "same kernel is the cross-check)")
    roof_mfma = None
    if "c5" in results:
        c5 = results["c5"]
        roof_mfma = dict(bound="mfma", kernel="wna16_prefill_kernel<128> (W13 with SwiGLU epilogue, C5)",
                         achieved=round(c5["w13_tflops"], 1), peak=BF16_PEAK_TFLOPS,
                         unit="TFLOP/s", frac=round(c5["w13_tflops"] / BF16_PEAK_TFLOPS, 4),
                         algorithmic_flops_per_launch=c5["w13_flops"],
                         launch_us=round(c5["w13_us"], 2),
                         w2_frac=round(c5["w2_tflops"] / BF16_PEAK_TFLOPS, 4),
                         layer_frac=round(c5["tflops"] / BF16_PEAK_TFLOPS, 4),
                         timing="HIP events around graph replays of the launch alone")
    line = dict(
        metric=METRIC, value=round(c3["layer_gbs"], 1), unit="GB/s", n_gpus=1, steps=args.steps,
        warmup=args.warmup, ms_per_step=round(c3["layer_us"] / 1e3, 5), higher_is_better=True,
        scaling="weak", vs_baseline=None, dtype="bf16",
        data="synthetic (seeded INT4 weights / bf16 N(0,1) activations / N(0,1) router logits)",
        config=dict(workload=c3["workload"], tokens=64, local_experts=48, hidden=7168, inter=2048,
                    topk=8, block_size=c3["block_size"], touched_experts=c3["touched_experts"],
                    launch=f"hip_graph ({GRAPH_LAYERS} layers per graph, each on its own "
                           "copy of the weights)",
                    layer_us_eager=round(c3["layer_us_eager"], 2),
                    layer_us=round(c3["layer_us"], 2),
                    layer_us_median=round(c3["layer_us_median"], 2),
                    layer_us_p99=round(c3["layer_us_p99"], 2),
                    layer_us_one_per_graph=round(c3["layer_us_one_per_graph"], 2),
                    algorithmic_bytes=c3["algorithmic_bytes"]),
        roofline=roof,
        roofline_prefill=roof_mfma,
        cpu_baseline=None if "cpu" not in results else {
            k: (round(v, 3) if isinstance(v, float) else v) for k, v in results["cpu"].items()},
        configs={k: v for k, v in results.items() if k not in ("cpu",)},
    )
    print(json.dumps(line))


if __name__ == "__main__":
    main()
