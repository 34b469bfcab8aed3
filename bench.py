"""Benchmark of the MI355X SRW layer (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload know]

A step is one SRW layer forward (``srw_forward`` through the C ABI) over the
workload's synthetic batch, inputs already resident in HBM.  The default
workload is the 40M Know pool named by the headline metric: T = 4096 tokens
(batch 8 x seq 512), d_model = 384, N = 25 200 units, score = x.E^T
(d_route = d_model), bf16, the reference's fused_gate_srw semantics
(models/dawn_spatial_v41_exp.py:415-635: one-pass moments of the bf16
scores, v4.1 gate, N chunked at 12 500 -> 2 chunks of 12 600).

Prints ONE JSON line (rank 0, N = 1) with the throughput, the roofline of
the dominant kernel (timed alone with HIP events that the library records
around it on the call's stream) and a CPU baseline: the oracle's
restatement of the same function timed on this host on a bounded sample of
the same workload.  Progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "SRW layer tokens/sec on 1 MI355X (40M Know pool); % bf16 MFMA / HBM peak"
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3        # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
# --cold: bytes written between timed calls, four times the 256 MB Infinity
# Cache (MALL), so that each call's pool reads come from HBM
COLD_FLUSH_BYTES = 1 << 30

# HBM bytes per launch of the dominant kernel: rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE (KiB per dispatch) scaled by what the same counters read for a
# 256 MiB copy (--calibrate-copy 256): FETCH x 2.00, WRITE x 1.00.  Keyed by
# (workload, stats mode, kernel family); profiles/know_T4096_N25200_traffic.md
# has the runs.
MEASURED_TRAFFIC = {
    # the scores-streaming main kernel: reads the 206 MB of bf16 scores the
    # moments kernel stored, besides R, W^T and x
    ("know", "onepass", "mfma_ss_bf16"): (133053.0 * 2.0 + 64575.2 * 1.0) * 1024,
    # profiles/decode_know_T64_N25200_kernel_stats.md
    ("decode_know", "onepass", "mfma_decode_bf16"): (22586.8 * 2.0 + 19709.4 * 1.0) * 1024,
}

WORKLOADS = {
    # name: (inputs.CONFIGS key, reference max_chunk_size, note)
    "know": ("know", 12500, "configs[0] Know pool at bf16 (the headline metric's 40M Know pool)"),
    "v": ("v", 12500, "configs[1] V pool"),
    "qk": ("qk", 12500, "configs[1] QK pool, paired routes sharing one x.R^T"),
    "decode_know": ("decode_know", 12500, "configs[3] decode-shaped Know pool, T=64, 3% pass"),
    "scaled": ("scaled", 12500, "configs[4] scaled Know pool d=1024 N=100000 T=16384, 2% pass"),
    # configs[1] as one layer's projections (its own branch below): the QK and V calls as one batch
    "qkv": (None, 12500, "configs[1] QK (paired) + V projections of one attention layer at T = 4096, "
                         "one srw_forward_batch"),
    # a whole decode step (its own branch below): 12 layers x (QK paired, V, Know) at T = 64
    "decode": (None, 12500, "configs[3] decode step: 64 single-token rows through the QK (paired), V and "
                            "Know pools for 12 layers, Know calibrated to 3% pass"),
    # the whole model (its own branch below): 12 layers, B = 32, S = 512, vocab 32 000
    "model": (None, 12500, "configs[2] full 12-layer DAWN-SRW 40M prefill forward (logits), the SRW "
                           "kernels timed inside it"),
}
MODEL_BATCH, MODEL_SEQ, MODEL_VOCAB = 32, 512, 32000


# Default run lengths, by GPU time: the clocks settle over the first ~70 ms
# of sustained load (a 0.34 ms step runs ~10 % slower in its first hundred
# launches than from the two-hundredth on), so the default warm-up covers
# that ramp and the timed region measures the sustained rate.
WARMUP_SECONDS = 0.3
TIMED_SECONDS = 1.0


def resolve_counts(args, run_once, sync) -> tuple[int, int]:
    """(warmup, steps): the explicit --warmup / --steps, or counts sized from
    one timed launch of ``run_once`` to WARMUP_SECONDS / TIMED_SECONDS."""
    if args.warmup is not None and args.steps is not None:
        return args.warmup, args.steps
    run_once()
    sync()
    t0 = time.perf_counter()
    run_once()
    sync()
    one = max(time.perf_counter() - t0, 1e-5)
    warmup = args.warmup if args.warmup is not None else max(5, int(WARMUP_SECONDS / one))
    steps = args.steps if args.steps is not None else min(5000, max(20, int(TIMED_SECONDS / one)))
    log(f"one step ~{one * 1e3:.3f} ms: warm-up {warmup} steps, {steps} timed")
    return warmup, steps


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# The CPU baseline runs on at most this many threads: a one-GPU box's share
# of the host's cores, whatever os.cpu_count() reports there.
CPU_THREADS_MAX = 16


def host_cpus() -> dict:
    """The host's logical CPU count beside the threads the baseline used
    ("cores"), so that a capped thread count is visible."""
    import torch
    return {"host_cpu_count": os.cpu_count(), "threads_used": torch.get_num_threads(),
            "thread_cap": CPU_THREADS_MAX}


def cpu_baseline(pkg, shape, inp, tau_value, chunk, budget_s: float, backward: bool = False,
                 f32_inference: bool = False, gate: str = "v41") -> dict:
    """The oracle's fused_gate_srw (bf16 emulation) -- or, with ``backward``,
    its hand-written VJP; with ``f32_inference`` its fp32 srw_inference;
    with ``gate`` "gelu_v401" the v4.0.1 forms of these -- on a token sample
    of the same pool, timed on the host cores (test infrastructure as the
    timed CPU restatement; never part of the GPU path)."""
    import torch
    from oracle import srw_ref, srw_vjp

    threads = torch.get_num_threads()
    T_s = min(shape.T, 1024)
    x = inp["x"][:T_s]
    tau = torch.full((T_s, shape.routes), tau_value)
    what = "fused_gate_srw"
    if backward and gate == "gelu_v401":
        what = "fused_gate_srw_gelu_v401 VJP (torch autograd through oracle/srw_ref.py)"
        bf = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
        h0 = x if shape.h_is_x else inp["h"][:T_s, 0]
        d_out = torch.randn(T_s, shape.D, generator=torch.Generator().manual_seed(1))

        def fn():
            xl, el, rl, wl = (bf(t).requires_grad_(True) for t in (x, inp["emb"], inp["read"], inp["write"]))
            hl = xl if shape.h_is_x else bf(h0).requires_grad_(True)
            tl = tau.clone().requires_grad_(True)
            res = srw_ref.fused_gate_srw_gelu_v401(xl[None], hl[None], el, tl[None], rl, wl, max_chunk_size=chunk)
            ((res[0][0] * d_out).sum() + 1e-2 * res[3]).backward()
    elif backward:
        what = "fused_gate_srw VJP (oracle/srw_vjp.py)"
        bf = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
        h = x if shape.h_is_x else inp["h"][:T_s, 0]
        d_out = torch.randn(T_s, shape.D, generator=torch.Generator().manual_seed(1))
        fn = lambda: srw_vjp.fused_gate_srw_vjp(  # noqa: E731
            bf(x), bf(h), bf(inp["emb"]), tau, bf(inp["read"]), bf(inp["write"]), d_out, 1e-2, 1e-2,
            max_chunk_size=chunk)
    elif f32_inference and shape.routes == 1:
        what = "srw_inference fp32"
        h = x if shape.h_is_x else inp["h"][:T_s, 0]
        ref_fn = srw_ref.srw_inference_gelu_v401 if gate == "gelu_v401" else srw_ref.srw_inference
        if gate == "gelu_v401":
            what = "srw_inference_gelu_v401 fp32"
        fn = lambda: ref_fn(x, h, inp["emb"], tau, inp["read"], inp["write"])  # noqa: E731
    elif gate == "gelu_v401":
        what = "fused_gate_srw_gelu_v401" + ("_paired" if shape.routes == 2 else "")
        if shape.routes == 1:
            h = x if shape.h_is_x else inp["h"][:T_s, 0]
            fn = lambda: srw_ref.fused_gate_srw_gelu_v401(  # noqa: E731
                x[None], h[None], inp["emb"], tau[None], inp["read"], inp["write"], max_chunk_size=chunk)
        else:
            h = inp["h"][:T_s]
            fn = lambda: srw_ref.fused_gate_srw_gelu_v401_paired(  # noqa: E731
                x[None], h[None], inp["emb"], tau.reshape(1, T_s, 2, 1), inp["read"], inp["write"],
                max_chunk_size=chunk)
    elif shape.routes == 1:
        h = x if shape.h_is_x else inp["h"][:T_s, 0]
        fn = lambda: srw_ref.fused_gate_srw(  # noqa: E731
            x[None], h[None], inp["emb"], tau[None], inp["read"], inp["write"],
            max_chunk_size=chunk)
    else:
        h = inp["h"][:T_s]
        fn = lambda: srw_ref.fused_gate_srw_paired(  # noqa: E731
            x[None], h[None], inp["emb"], tau.reshape(1, T_s, 2, 1), inp["read"],
            inp["write"], max_chunk_size=chunk)
    fn()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    log(f"cpu baseline: T_sample={T_s} runs={len(times)} median={med * 1e3:.1f} ms "
        f"threads={threads}")
    return {"value": T_s / med, "unit": "tokens/s", "cores": threads, "kind": "port",
            **host_cpus(),
            "sample": (f"oracle {what}{'' if f32_inference else ' bf16 emulation'}, first {T_s} of the "
                       f"{shape.T} tokens, full pool N={shape.N}, median of {len(times)} "
                       f"runs; {cpu_model()}")}


DECODE_LAYERS = 12


def bench_decode(args, pkg, C, dev) -> dict:
    """one decode step = 12 layers x three SRW calls (the QK pool
    with its paired routes, V, Know) on 64 rows, the pools shared by the
    layers (v41:1393-1394), router h = x W + b with d_route 128, the Know
    tau_offset calibrated to ~3 % pass; per layer the QK and V calls as one
    srw_forward_batch.  Captured once as a HIP graph and replayed.  The dominant kernel is the Know pool's decode kernel (timed by
    an eager call after the replays)."""
    import torch
    bf = torch.bfloat16
    plans, shapes = [], []
    for key in ("decode_qk", "decode_v", "decode_know"):
        shape = pkg.inputs.CONFIGS[key]
        inp = pkg.inputs.make_pool_inputs(shape, seed=args.seed)
        if shape.pass_target is not None:
            inp["tau_offset"].fill_(pkg.inputs.calibrate_tau_offset(inp, shape.pass_target))
        _, cs = pkg.chunk_plan(shape.N, 12500)
        plan = pkg.SrwPlan(inp["x"].to(bf).to(dev), inp["h"].to(bf).to(dev), inp["emb"].to(bf).to(dev),
                           inp["tau_offset"].to(dev), inp["read"].to(bf).to(dev), inp["write"].to(bf).to(dev),
                           stats=args.stats, chunk_size=cs, want_mask=True)
        plans.append(plan)
        shapes.append(shape)
    stream = torch.cuda.current_stream(dev)
    for pl in plans:
        pl.launch(stream)
    # the QK and V calls of a layer read the same input: one srw_forward_batch
    # (one launch per stage); the Know call follows the attention, on its own
    qkv = pkg.SrwBatchPlan(plans[:2])
    qkv.launch(stream)
    torch.cuda.synchronize()
    log("decode paths: " + ", ".join(f"{s_.note.split(':')[1].strip()} -> {pl.path}"
                                     for s_, pl in zip(shapes, plans)))

    def step(st):
        for _ in range(DECODE_LAYERS):
            qkv.launch(st, pool_cached=True)
            plans[2].launch(st, pool_cached=True)

    cap = torch.cuda.Stream(dev)
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        step(cap)
    stream.wait_stream(cap)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        step(cap)
    torch.cuda.synchronize()
    warmup, K = resolve_counts(args, graph.replay, torch.cuda.synchronize)
    t_begin = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    t_begin.record(stream)
    t_end.record(stream)
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t_begin.record(stream)
    for _ in range(K):
        graph.replay()
    t_end.record(stream)
    torch.cuda.synchronize()
    step_ms = t_begin.elapsed_time(t_end) / K
    # the Know decode kernel alone, eagerly
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
    for a, b in ev:
        a.record(stream)
        b.record(stream)
    torch.cuda.synchronize()
    for a, b in ev:
        C.set_kernel_events(a.cuda_event, b.cuda_event)
        plans[2].launch(stream, pool_cached=True)
    torch.cuda.synchronize()
    C.set_kernel_events(None, None)
    kern_ms = statistics.mean(a.elapsed_time(b) for a, b in ev)
    pool_bytes = [s_.N * (s_.dr + 2 * s_.D) * 2 for s_ in shapes]
    step_bytes = DECODE_LAYERS * sum(pool_bytes)
    log(f"timed {K} decode steps ({DECODE_LAYERS} layers x 3 pools): {step_ms:.4f} ms/step, "
        f"Know kernel {kern_ms:.4f} ms, pool stream {step_bytes / (step_ms * 1e-3) / 1e9:.0f} GB/s")
    achieved = pool_bytes[2] / (kern_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": None, "kernel": plans[2].path, "kernel_ms": round(kern_ms, 5),
                "algorithmic_bytes": pool_bytes[2],
                "step_pool_bytes": step_bytes,
                "step_gbs": round(step_bytes / (step_ms * 1e-3) / 1e9, 1)}
    cpu = None
    if args.cpu_seconds > 0:
        from oracle import srw_ref
        torch.set_num_threads(min(os.cpu_count() or 1, CPU_THREADS_MAX))
        t0 = time.perf_counter()
        for pl, s_ in zip(plans, shapes):
            x, h, emb, tau, read, write = (t.float().cpu() for t in pl.inputs)
            if s_.routes == 2:
                srw_ref.fused_gate_srw_paired(x[None], h[None], emb, tau.reshape(1, s_.T, 2, 1), read, write,
                                              max_chunk_size=12500)
            else:
                srw_ref.fused_gate_srw(x[None], h[:, 0][None], emb, tau[None], read, write, max_chunk_size=12500)
        layer_s = time.perf_counter() - t0
        log(f"cpu baseline: one layer (3 pools, 64 rows) {layer_s:.2f} s")
        cpu = {"value": 64 / (layer_s * DECODE_LAYERS), "unit": "tokens/s", "cores": torch.get_num_threads(),
               "kind": "port", **host_cpus(),
               "sample": (f"oracle fused_gate_srw / _paired (bf16 emulation) of one of the {DECODE_LAYERS} layers "
                          f"(QK, V, Know at 64 rows), scaled to {DECODE_LAYERS} layers; {cpu_model()}")}
    return {
        "metric": METRIC, "value": round(64 / (step_ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": K, "warmup": warmup, "ms_per_step": round(step_ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x RMS-normalised; router h = x W + b; E, R, W unit rows)",
        "config": {"workload": "decode", "note": WORKLOADS["decode"][2], "T": 64, "layers": DECODE_LAYERS,
                   "pools": {s_.note.split(":")[1].strip(): s_.N for s_ in shapes}, "d_model": 384,
                   "d_route": 128, "stats": args.stats, "graph": True, "pool_cached": True, "qk_v_batched": True,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }


def bench_qkv(args, pkg, C, dev) -> dict:
    """Q, K and V of one attention layer at T = 4096 -- the QK
    pool's paired call and the V pool's call, issued as one
    srw_forward_batch (one launch per stage).  The dominant kernel is the
    batch's main kernel (both calls' workgroups)."""
    import torch
    bf = torch.bfloat16
    plans, shapes = [], []
    for key in ("qk", "v"):
        shape = pkg.inputs.CONFIGS[key]
        inp = pkg.inputs.make_pool_inputs(shape, seed=args.seed)
        _, cs = pkg.chunk_plan(shape.N, 12500)
        x = inp["x"].to(bf).to(dev)
        h = x if shape.h_is_x else inp["h"].to(bf).to(dev)
        plans.append(pkg.SrwPlan(x, h, inp["emb"].to(bf).to(dev), inp["tau_offset"].to(dev),
                                 inp["read"].to(bf).to(dev), inp["write"].to(bf).to(dev),
                                 stats=args.stats, chunk_size=cs, want_mask=True))
        shapes.append(shape)
    stream = torch.cuda.current_stream(dev)
    batch = pkg.SrwBatchPlan(plans)
    batch.launch(stream)
    torch.cuda.synchronize()
    log(f"qkv path: {batch.path}")

    def step():
        batch.launch(stream, pool_cached=args.pool_cached)

    warmup, K = resolve_counts(args, step, torch.cuda.synchronize)
    ev_k = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    t_begin = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    for a, b in ev_k + [(t_begin, t_end)]:
        a.record(stream)
        b.record(stream)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t_begin.record(stream)
    for i in range(K):
        C.set_kernel_events(ev_k[i][0].cuda_event, ev_k[i][1].cuda_event)
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    C.set_kernel_events(None, None)
    step_ms = t_begin.elapsed_time(t_end) / K
    kern_ms = statistics.mean(a.elapsed_time(b) for a, b in ev_k)
    T = shapes[0].T
    log(f"timed {K} steps (QK + V): {step_ms:.4f} ms/step, batch main kernel {kern_ms:.4f} ms")
    # The roofline needs the batch's one main kernel: when the calls fell
    # back to running one after the other, every call re-recorded the events
    # and they bracket only the last call's main kernel.
    roofline = None
    if batch.path == "mfma_batch_bf16":
        # the streaming main kernel leaves the score GEMM to the moments kernel
        ss = all(s_.dr >= s_.D for s_ in shapes)
        kflops = sum(2.0 * T * s_.N * ((0 if ss else s_.routes * s_.dr) + s_.D + s_.routes * s_.D)
                     for s_ in shapes)
        achieved = kflops / (kern_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
                    "kernel": batch.path, "kernel_ms": round(kern_ms, 5), "algorithmic_flop": kflops}
    else:
        log(f"qkv: the calls ran one after the other (path {batch.path}); no single main kernel, "
            "roofline null")
    cpu = None
    if args.cpu_seconds > 0:
        cpu = qkv_cpu_baseline(pkg, shapes, args.seed, args.cpu_seconds)
    return {
        "metric": METRIC, "value": round(T / (step_ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": K, "warmup": warmup, "ms_per_step": round(step_ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x RMS-normalised; E ~ N(0,1/dr); R, W L2-normalised rows)",
        "config": {"workload": "qkv", "note": WORKLOADS["qkv"][2], "T": T, "d_model": 384, "d_route": 384,
                   "pools": {"qk": shapes[0].N, "v": shapes[1].N}, "stats": args.stats,
                   "pool_cached": args.pool_cached, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }


def qkv_cpu_baseline(pkg, shapes, seed, budget_s: float) -> dict:
    """configs[1] on the host: the oracle's fused_gate_srw_paired (QK pool)
    and fused_gate_srw (V pool) -- the reference's two calls of one layer,
    v41:1036-1053 -- on the first 512 of the 4096 tokens of the same seeded
    inputs, bf16 emulation (test infrastructure timed as the CPU
    restatement; never part of the GPU path)."""
    import torch
    from oracle import srw_ref
    torch.set_num_threads(min(os.cpu_count() or 1, CPU_THREADS_MAX))
    T_s = min(shapes[0].T, 512)
    qk = pkg.inputs.make_pool_inputs(shapes[0], seed=seed, T=T_s)
    v = pkg.inputs.make_pool_inputs(shapes[1], seed=seed, T=T_s)

    def fn():
        srw_ref.fused_gate_srw_paired(qk["x"][None], qk["h"][None], qk["emb"],
                                      qk["tau_offset"].reshape(1, T_s, 2, 1), qk["read"], qk["write"],
                                      max_chunk_size=12500)
        srw_ref.fused_gate_srw(v["x"][None], v["x"][None], v["emb"], v["tau_offset"][None], v["read"],
                               v["write"], max_chunk_size=12500)

    fn()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    log(f"cpu baseline (qkv): T_sample={T_s} runs={len(times)} median={med * 1e3:.1f} ms "
        f"threads={torch.get_num_threads()}")
    return {"value": T_s / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            **host_cpus(),
            "sample": (f"oracle fused_gate_srw_paired (QK, N={shapes[0].N}) + fused_gate_srw (V, "
                       f"N={shapes[1].N}), bf16 emulation, first {T_s} of the {shapes[0].T} tokens, "
                       f"median of {len(times)} runs; {cpu_model()}")}


def bench_model(args, pkg, C, dev) -> dict:
    """DAWN.__call__ (deterministic) over B x S uniform token ids
    with random-init weights of the 40M architecture; a step is one forward
    to the logits.  The dominant kernel is the Know pool's fused SRW kernel
    (the last layer's call of each step is the one timed)."""
    import torch
    cfg = pkg.DawnConfig(vocab_size=MODEL_VOCAB)
    B, S = MODEL_BATCH, MODEL_SEQ
    T, D, dr, L = B * S, cfg.d_model, cfg.d_route, cfg.n_layers
    params = pkg.init_params(cfg, seed=args.seed)
    model = pkg.DawnModel(params, cfg, dev)
    ids = torch.randint(0, cfg.vocab_size, (B, S), generator=torch.Generator().manual_seed(args.seed))
    ids_dev = ids.to(dev)
    stream = torch.cuda.current_stream(dev)
    model.forward(ids_dev)
    torch.cuda.synchronize()
    log(f"model built: T={T}, paths " + ", ".join(
        f"{k[0]}:{c.plan.path}" for k, c in model._calls.items()))
    warmup, K = resolve_counts(args, lambda: model.forward(ids_dev), torch.cuda.synchronize)
    ev_k = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(K)]
    for a, b in ev_k:
        a.record(stream)
        b.record(stream)
    t_begin = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    t_begin.record(stream)
    t_end.record(stream)
    for _ in range(warmup):
        model.forward(ids_dev)
    torch.cuda.synchronize()
    t_begin.record(stream)
    for i in range(K):
        C.set_kernel_events(ev_k[i][0].cuda_event, ev_k[i][1].cuda_event)
        model.forward(ids_dev)
    t_end.record(stream)
    torch.cuda.synchronize()
    C.set_kernel_events(None, None)
    step_ms = t_begin.elapsed_time(t_end) / K
    kern_ms = statistics.mean(a.elapsed_time(b) for a, b in ev_k)
    log(f"timed {K} forwards: {step_ms:.3f} ms/step, Know kernel {kern_ms:.4f} ms")
    srw = L * 2.0 * T * (cfg.n_qk * (2 * dr + 3 * D) + cfg.n_v * (dr + 2 * D) + cfg.n_know * (dr + 2 * D))
    glue = (L * (2.0 * T * D * (4 * dr + 4) + 2.0 * T * D * D + 4.0 * B * S * S * D)
            + 2.0 * T * D * cfg.vocab_size)
    know_path = model._calls[("know", T, 1, "onepass")].plan.path
    # the Know call's main kernel; the scores-streaming one leaves the score GEMM to the moments kernel
    kflops = 2.0 * T * cfg.n_know * ((0 if know_path == "mfma_ss_bf16" else dr) + 2 * D)
    achieved = kflops / (kern_ms * 1e-3) / 1e12
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
                "kernel": know_path,
                "kernel_ms": round(kern_ms, 5), "algorithmic_flop": kflops,
                "step_tflops": round((srw + glue) / (step_ms * 1e-3) / 1e12, 2),
                "srw_flop_per_step": srw, "glue_flop_per_step": glue}
    cpu = None
    if args.cpu_seconds > 0:
        from oracle import dawn_ref
        torch.set_num_threads(min(os.cpu_count() or 1, CPU_THREADS_MAX))
        S_s = 64
        sample = ids[:1, :S_s]
        times = []
        t0 = time.perf_counter()
        while not times or (time.perf_counter() - t0 < args.cpu_seconds and len(times) < 5):
            t1 = time.perf_counter()
            dawn_ref.forward(params, cfg, sample)
            times.append(time.perf_counter() - t1)
        med = statistics.median(times)
        log(f"cpu baseline: {S_s} tokens, runs={len(times)} median={med:.2f} s")
        cpu = {"value": S_s / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               **host_cpus(),
               "sample": (f"oracle DAWN forward (oracle/dawn_ref.py, bf16-emulated SRW, f32 glue), "
                          f"1 x {S_s} tokens of the same ids, full 40M model, median of {len(times)} "
                          f"runs; {cpu_model()}")}
    return {
        "metric": METRIC, "value": round(T / (step_ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": K, "warmup": warmup, "ms_per_step": round(step_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": ("synthetic (token ids uniform over the vocabulary, seeded; random-init weights "
                 "with the reference's initialisers)"),
        "config": {"workload": "model", "note": WORKLOADS["model"][2], "batch": B, "seq_len": S,
                   "tokens": T, "n_layers": L, "d_model": D, "d_route": dr, "n_heads": cfg.n_heads,
                   "vocab": cfg.vocab_size, "pools": [cfg.n_qk, cfg.n_v, cfg.n_know],
                   "srw": "bf16, one-pass statistics, chunk 12500", "glue": "float32",
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }


def sparse_accounting(plan, T, D, dr, N, R, path, cs=None):
    """What SRW_FLAG_SPARSE_SKIP can leave out, from the call's pass mask.

    Decode kernel (path mfma_decode_sparse_bf16): a unit's R row (D bf16) is
    read when some row of the call passes it, a W^T fragment half (8 units,
    D / 32 pieces of 512 bytes) when one of its units passes; E is read
    whole.  Tiled family (path tiled_sparse_bf16): per 32-row tile the read
    and write GEMMs run over the union of the units some row of the tile
    passes, in blocks of 32 listed units that never cross a reference chunk
    (cs units): executed_flop counts those blocks (4 * 32 * 32 * D each),
    dense_flop the dense read + write GEMMs, pass_pair_flop the (row, unit)
    pairs that pass.  Other prefill shapes run dense: reported is the share
    of 32-token x 32-unit blocks no row passes (what a block skip could drop).
    """
    import torch
    words = plan.pass_mask.reshape(T * R, -1)                                  # [rows, ceil(N/64)] 64-bit words
    info = {"pass_frac": round(float(plan.n_active.double().sum()) / (T * R * N), 5)}
    if path == "tiled_sparse_bf16":
        rows = T * R
        tb = (rows + 31) // 32
        pad = torch.zeros(tb * 32, words.shape[1], dtype=words.dtype, device=words.device)
        pad[:rows] = words
        blk = pad.reshape(tb, 32, -1)
        ored = blk[:, 0].clone()
        for i in range(1, 32):                                                 # OR over each 32-row tile
            ored |= blk[:, i]
        shifts = torch.arange(64, device=ored.device)
        uni = ((ored.unsqueeze(-1) >> shifts) & 1).reshape(tb, -1)[:, :N].to(torch.int32)   # [tiles, N]
        cs = cs or N
        bounds = list(range(0, N, cs)) + [N]
        counts = torch.stack([uni[:, a:b].sum(dim=1) for a, b in zip(bounds[:-1], bounds[1:])], dim=1)
        blocks = int(((counts + 31) // 32).sum())
        listed = int(counts.sum())
        info.update({"union_frac": round(listed / (tb * N), 5),
                     "listed_units_per_tile": round(listed / tb, 1),
                     "executed_flop": 4.0 * 32 * 32 * D * blocks,
                     "dense_flop": 4.0 * rows * N * D,
                     "pass_pair_flop": 4.0 * D * float(plan.n_active.double().sum())})
    elif path == "mfma_decode_sparse_bf16":
        anyw = words[0].clone()
        for r in range(1, T * R):                                              # OR over the call's rows
            anyw |= words[r]
        act = ((anyw.unsqueeze(-1) >> torch.arange(64, device=anyw.device)) & 1).reshape(-1)[:N].bool()
        ntiles = (N + 31) // 32
        pad = torch.zeros(ntiles * 32, dtype=torch.bool, device=act.device)
        pad[:N] = act
        t = pad.reshape(ntiles, 2, 2, 2, 4)                                    # [tile][j][run][half][4]
        halves = t.any(dim=-1).any(dim=2)                                      # [tile][j][half]
        need = N * dr * 2 + int(act.sum()) * D * 2 + int(halves.sum()) * (D // 32) * 512
        info.update({"active_units_frac": round(float(act.float().mean()), 5),
                     "w_halves_read_frac": round(float(halves.float().mean()), 5),
                     "needed_bytes": need, "pool_bytes": N * (dr + 2 * D) * 2})
    else:
        rows = T * R
        tb = (rows + 31) // 32
        pad = torch.zeros(tb * 32, words.shape[1], dtype=words.dtype, device=words.device)
        pad[:rows] = words
        blk = pad.reshape(tb, 32, -1)
        ored = blk[:, 0].clone()
        for i in range(1, 32):                                                 # OR over each 32-row block
            ored |= blk[:, i]
        lo_half = (ored & 0xFFFFFFFF) != 0                                     # units 64 w .. 64 w + 31
        hi_half = (ored >> 32) != 0                                            # units 64 w + 32 .. 64 w + 63
        n_ub = (N + 31) // 32
        busy = torch.stack([lo_half, hi_half], dim=-1).reshape(tb, -1)[:, :n_ub]
        info.update({"note": "no sparse kernel for this shape (more than 128 rows): run dense",
                     "skippable_block_frac": round(1.0 - float(busy.float().mean()), 6)})
    return info


def time_dense_twin(args, pkg, C, plan, cs, stream, K, warmup, sparse_step_ms, T, R, N, D):
    """The same call without SRW_FLAG_SPARSE_SKIP (the dense tiled kernels),
    timed like the sparse one: its step, its dominant kernel (the gate
    kernel: read GEMM + gate) and the write GEMM's share of the read + write
    work it does densely."""
    import torch
    x, h, emb, tau, read, write = plan.inputs
    dense = pkg.SrwPlan(x, h, emb, tau, read, write, stats=args.stats, chunk_size=cs, want_mask=True,
                        tiled=args.tiled, sparse_skip=False, gate=args.gate)
    for _ in range(warmup):
        dense.launch(stream)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(K)]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for a, b in ev + [(t0, t1)]:      # materialise the HIP events on this stream
        a.record(stream)
        b.record(stream)
    torch.cuda.synchronize()
    t0.record(stream)
    for a, b in ev:
        C.set_kernel_events(a.cuda_event, b.cuda_event)
        dense.launch(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    C.set_kernel_events(None, None)
    step_ms = t0.elapsed_time(t1) / K
    kern_ms = statistics.mean(a.elapsed_time(b) for a, b in ev)
    same = bool(torch.equal(dense.n_active, plan.n_active) and torch.equal(dense.den, plan.den))
    kflops = 2.0 * T * R * N * D
    log(f"dense twin ({dense.path}): {step_ms:.4f} ms/step, gate kernel {kern_ms:.4f} ms")
    return {"path": dense.path, "ms_per_step": round(step_ms, 5), "kernel": "tiled_gate_kernel",
            "kernel_ms": round(kern_ms, 5),
            "kernel_mfma_frac": round(kflops / (kern_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "step_speedup_of_sparse": round(step_ms / sparse_step_ms, 3),
            "same_n_active_and_den": same}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: as many as take about %.0f s)" % TIMED_SECONDS)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default: as many as take about %.1f s)" % WARMUP_SECONDS)
    ap.add_argument("--workload", default="know", choices=sorted(WORKLOADS))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--stats", default="onepass", choices=["onepass", "centered", "gram"])
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="time budget of the CPU baseline (0 skips it)")
    ap.add_argument("--force-generic", action="store_true",
                    help="time the generic (scalar) kernels instead of the MFMA path")
    ap.add_argument("--tiled", action="store_true",
                    help="run the tiled-GEMM kernels (P materialised) where a fused kernel "
                         "exists too (they serve d_model > 384 anyway)")
    ap.add_argument("--no-residuals", action="store_true",
                    help="with --backward: no forward residuals (den, unit statistics); the "
                         "backward recomputes them from the scores")
    ap.add_argument("--backward", action="store_true",
                    help="time the backward (srw_backward: the VJP of fused_gate_srw for the "
                         "training step) instead of the forward; one route, bf16")
    ap.add_argument("--diag", action="store_true",
                    help="also compute the training diagnostics (SRW_FLAG_DIAG: the 22-tuple "
                         "path of the drop-in fused_gate_srw)")
    ap.add_argument("--pool-cached", action="store_true",
                    help="steps after the first reuse the pool data kept in the workspace "
                         "(SRW_FLAG_POOL_CACHED: decode steps / layers sharing one pool)")
    ap.add_argument("--sparse", action="store_true",
                    help="SRW_FLAG_SPARSE_SKIP: the decode kernel loads only the R rows and W^T fragment "
                         "halves of units some row passes (the roofline counts the bytes it needs); the "
                         "tiled family (d_model 256 / 512 / 1024) runs the read and write GEMMs over each "
                         "32-token tile's passing units (the roofline counts the executed MFMA work, and "
                         "the same call without the flag is timed beside it); other prefill shapes run "
                         "dense (the line reports how many 32x32 (token, unit) blocks a skip could drop)")
    ap.add_argument("--tokens", type=int, default=0,
                    help="override the workload's token count (e.g. 1 or 8 rows for a decode shape)")
    ap.add_argument("--gate", default="v41", choices=["v41", "gelu_v401"],
                    help="v4.1 gate (default) or the v4.0.1 GELU gate")
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "f32"],
                    help="operand dtype of the single-pool workloads (f32: the fp32 matrix-core "
                         "family; configs[0] as written is f32 with --stats centered)")
    ap.add_argument("--cold", action="store_true",
                    help="write 1 GiB between timed calls (evicting the Infinity Cache and the L2s) "
                         "and time each call on its own: pool reads from HBM")
    ap.add_argument("--graph", action="store_true",
                    help="capture one call in a HIP graph and time graph replays (launch-bound "
                         "shapes such as decode)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                    help="first run one device-to-device copy of MB MiB (a known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    if args.backward and (args.graph or args.diag or args.stats != "onepass"):
        print("bench.py: --backward times srw_backward (one-pass statistics, no graph, no "
              "diagnostics)", file=sys.stderr)
        return 2
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs the SRW layer on one GPU only; "
              "--gpus above 1 is not supported (token-sharding design is documented, "
              "not built)", file=sys.stderr)
        return 2

    import torch
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    from dawn_srw_amd import _capi as C

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.dtype == "f32" and (args.workload in ("decode", "qkv", "model") or args.backward or args.tiled):
        print("bench.py: --dtype f32 times the single-pool forward", file=sys.stderr)
        return 2
    if args.gate != "v41" and args.workload in ("decode", "qkv", "model"):
        print("bench.py: --gate gelu_v401 times the single-pool calls", file=sys.stderr)
        return 2
    if args.cold and (args.graph or args.workload in ("decode", "qkv", "model")):
        print("bench.py: --cold times single eager calls of one pool", file=sys.stderr)
        return 2
    if args.workload == "decode":
        if args.backward or args.diag or args.tiled:
            print("bench.py: --workload decode times the forward decode step", file=sys.stderr)
            return 2
        print(json.dumps(bench_decode(args, pkg, C, dev)), flush=True)
        return 0
    if args.workload == "qkv":
        if args.backward or args.graph or args.diag or args.tiled:
            print("bench.py: --workload qkv times the batched forward", file=sys.stderr)
            return 2
        print(json.dumps(bench_qkv(args, pkg, C, dev)), flush=True)
        return 0
    if args.workload == "model":
        if args.backward or args.graph or args.diag or args.tiled or args.stats != "onepass":
            print("bench.py: --workload model times the plain forward", file=sys.stderr)
            return 2
        print(json.dumps(bench_model(args, pkg, C, dev)), flush=True)
        return 0
    key, max_chunk, note = WORKLOADS[args.workload]
    shape = pkg.inputs.CONFIGS[key]
    if args.tokens > 0:
        import dataclasses
        shape = dataclasses.replace(shape, T=args.tokens)
        note += f" (T overridden to {args.tokens})"
    _, cs = pkg.chunk_plan(shape.N, max_chunk)
    log(f"workload {args.workload}: T={shape.T} D={shape.D} dr={shape.dr} N={shape.N} "
        f"R={shape.routes} chunk={cs}")

    if args.calibrate_copy > 0:
        n = args.calibrate_copy * (1 << 20) // 4
        # a source no kernel has written, so that its reads come from HBM
        src = torch.empty(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration copy: {args.calibrate_copy} MiB read + {args.calibrate_copy} MiB written")
        del src, dst

    inp = pkg.inputs.make_pool_inputs(shape, seed=args.seed)
    tau_value = -0.5
    if shape.pass_target is not None:
        tau_value = pkg.inputs.calibrate_tau_offset(inp, shape.pass_target)
        inp["tau_offset"].fill_(tau_value)
    bf = torch.float32 if args.dtype == "f32" else torch.bfloat16
    x = inp["x"].to(bf).to(dev)
    h = x if shape.h_is_x else inp["h"].to(bf).to(dev)
    plan = pkg.SrwPlan(x, h, inp["emb"].to(bf).to(dev), inp["tau_offset"].to(dev),
                       inp["read"].to(bf).to(dev), inp["write"].to(bf).to(dev),
                       stats=args.stats, chunk_size=cs, want_mask=True, diag=args.diag,
                       force_generic=args.force_generic, tiled=args.tiled, sparse_skip=args.sparse,
                       gate=args.gate)
    stream = torch.cuda.current_stream(dev)

    plan.launch(stream)
    torch.cuda.synchronize()
    log(f"first call done, path={plan.path}, mean active/token="
        f"{plan.n_active.float().mean().item():.1f}")

    def step():
        plan.launch(stream, pool_cached=args.pool_cached)

    if args.backward:
        # cotangents of out (synthetic, seeded) and of score_lb / dead_penalty
        gen = torch.Generator().manual_seed(args.seed + 1)
        d_out = torch.randn(shape.T, 1, shape.D, generator=gen).to(dev)
        den = unit_diag = None
        if not args.no_residuals:
            # the drop-in's training path: its forward (with diagnostics)
            # hands the backward its den and unit statistics
            fplan = pkg.SrwPlan(*plan.inputs[:6], stats=args.stats, chunk_size=cs, want_mask=False, diag=True,
                                gate=args.gate)
            fplan.launch(stream)
            torch.cuda.synchronize()
            den, unit_diag = fplan.den, fplan.unit_diag
        # the v4.0.1 function has no dead_penalty (its cotangent stays 0)
        d_pen = 0.0 if args.gate == "gelu_v401" else 1e-2
        bplan = pkg.SrwBackwardPlan(x, h, plan.inputs[2], plan.inputs[3], plan.inputs[4],
                                    plan.inputs[5], plan.out, d_out, 1e-2, d_pen, den=den, unit_diag=unit_diag,
                                    gate=args.gate)
        bplan.launch(stream)
        torch.cuda.synchronize()
        log(f"backward first call done, path={bplan.path}, workspace {bplan.ws_bytes / 2**30:.2f} GiB")

        def step():  # noqa: F811
            bplan.launch(stream)

    graph = None
    if args.graph:
        # a side stream for capture, as torch requires; replays run on `stream`
        cap = torch.cuda.Stream(dev)
        cap.wait_stream(stream)
        with torch.cuda.stream(cap):
            plan.launch(cap, pool_cached=args.pool_cached)
        stream.wait_stream(cap)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            plan.launch(cap, pool_cached=args.pool_cached)
        torch.cuda.synchronize()
        log("captured one call in a HIP graph")

    run_once = graph.replay if graph is not None else step
    warmup, K = resolve_counts(args, run_once, torch.cuda.synchronize)
    ev_k = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(K)]
    t_begin = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    for a, b in ev_k + [(t_begin, t_end)]:      # materialise the HIP events on this stream
        a.record(stream)
        b.record(stream)
    # the warm-up runs straight into the timed region (one synchronize between)
    for _ in range(warmup):
        run_once()
    torch.cuda.synchronize()
    if args.cold:
        # each call timed on its own, after 1 GiB of writes: no pool line left
        # in the Infinity Cache or an L2
        flush = torch.empty(COLD_FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
        ev_call = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(K)]
        torch.cuda.synchronize()
        wall0 = time.perf_counter()
        for i in range(K):
            flush.fill_(float(i))
            flush.sum()   # read back: the cache then holds clean flush lines, no dirty ones to evict
            ev_call[i][0].record(stream)
            C.set_kernel_events(ev_k[i][0].cuda_event, ev_k[i][1].cuda_event)
            step()
            ev_call[i][1].record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        C.set_kernel_events(None, None)
        step_ms = statistics.mean(a.elapsed_time(b) for a, b in ev_call)
        del flush
    else:
        wall0 = time.perf_counter()
        t_begin.record(stream)
        for i in range(K):
            if graph is not None:
                graph.replay()
                continue
            C.set_kernel_events(ev_k[i][0].cuda_event, ev_k[i][1].cuda_event)
            step()
        t_end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        C.set_kernel_events(None, None)
        step_ms = t_begin.elapsed_time(t_end) / K
    if graph is not None:
        # the dominant kernel's own events are not recorded inside a replay:
        # time it eagerly once more
        ev_k = ev_k[:200]
        for a, b in ev_k:
            C.set_kernel_events(a.cuda_event, b.cuda_event)
            step()
        torch.cuda.synchronize()
        C.set_kernel_events(None, None)
    kern_ms = statistics.mean(a.elapsed_time(b) for a, b in ev_k)
    log(f"timed {K} steps: {step_ms:.4f} ms/step (events), wall {wall / K * 1e3:.4f} ms/step, "
        f"dominant kernel {kern_ms:.4f} ms")

    T, D, dr, N, R = shape.T, shape.D, shape.dr, shape.N, shape.routes
    flops = 2.0 * T * N * (R * dr + D + R * D)          # score + read (once) + write
    path = bplan.path if args.backward else plan.path
    if args.backward:
        # recompute (score + read), dP, dW, dR, dx (d_model) and dE, dh (d_route)
        flops = 2.0 * T * N * (3 * dr + 5 * D)
        kflops = 2.0 * T * N * D        # the dominant kernel: dP = draw . W^T with the gate derivative
    elif plan.path == "mfma_ss_bf16":
        # the main kernel streams the moments kernel's bf16 scores: its own
        # work is the read (once per token) and write GEMMs
        kflops = 2.0 * T * N * (D + R * D)
    elif plan.path == "tiled_sparse_bf16":
        kflops = None   # the gather kernel's executed MFMA work, from the pass mask below
    elif plan.path in ("tiled_bf16", "tiled_f32"):
        # the dominant kernel of the tiled family is tiled_gate_kernel: the
        # read GEMM over the T * R virtual rows, gating the scores that
        # tiled_stats_kernel stored (the score and write GEMMs are kernels of
        # their own)
        kflops = 2.0 * T * R * N * D
    else:
        kflops = flops
    sparse_info = None
    if args.sparse and not args.backward:
        sparse_info = sparse_accounting(plan, T, D, dr, N, R, path, cs)
        if path == "tiled_sparse_bf16":
            # sp_gather_kernel: the read and write GEMMs over the listed blocks
            kflops = sparse_info["executed_flop"]
            sparse_info["dense_equivalent_tflops"] = round(sparse_info["dense_flop"] / (kern_ms * 1e-3) / 1e12, 2)
            sparse_info["dense"] = time_dense_twin(args, pkg, C, plan, cs, stream, K, warmup, step_ms, T, R, N, D)
    achieved = kflops / (kern_ms * 1e-3) / 1e12
    traffic = MEASURED_TRAFFIC.get((args.workload, args.stats, path))
    peak = PEAK_F32_TFLOPS if args.dtype == "f32" else PEAK_BF16_TFLOPS
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
                "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                "traffic": traffic, "kernel": path,
                "kernel_ms": round(kern_ms, 5), "algorithmic_flop": kflops,
                "step_tflops": round(flops / (step_ms * 1e-3) / 1e12, 2)}
    if args.workload.startswith("decode_") and not args.backward:
        # decode shapes are pool-read bound: the algorithmic bytes are the pool
        # (E, R, W rows) streamed once per call -- with the sparse kernel the
        # E rows and the R rows / W^T halves of units some row passes
        pool_bytes = N * (dr + 2 * D) * 2
        need = sparse_info["needed_bytes"] if (sparse_info and "needed_bytes" in sparse_info) else pool_bytes
        gbs = need / (kern_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "kernel": path,
                    "kernel_ms": round(kern_ms, 5), "algorithmic_bytes": need,
                    "step_gbs": round(need / (step_ms * 1e-3) / 1e9, 1)}
        if sparse_info is not None:
            roofline["dense_equivalent_gbs"] = round(pool_bytes / (kern_ms * 1e-3) / 1e9, 1)
    if sparse_info is not None:
        roofline["sparse"] = sparse_info

    cpu = None
    if args.cpu_seconds > 0:
        torch.set_num_threads(min(os.cpu_count() or 1, CPU_THREADS_MAX))
        cpu = cpu_baseline(pkg, shape, inp, tau_value, max_chunk, args.cpu_seconds, args.backward,
                           f32_inference=args.dtype == "f32" and args.stats == "centered", gate=args.gate)

    value = T / (step_ms * 1e-3)
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": K, "warmup": warmup, "ms_per_step": round(step_ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": args.dtype, "data": "synthetic (seeded N(0,1) x RMS-normalised; E ~ N(0,1/dr); "
                                  "R, W L2-normalised rows)",
        "config": {"workload": args.workload, "note": note, "T": T, "d_model": D,
                   "d_route": dr, "n_units": N, "routes": R, "chunk": cs,
                   "stats": args.stats, "diag": args.diag, "pool_cached": args.pool_cached,
                   "tiled": args.tiled, "pass": "backward" if args.backward else "forward",
                   "residuals": bool(args.backward and not args.no_residuals),
                   "graph": args.graph, "sparse_skip": args.sparse, "gate": args.gate,
                   "cold": args.cold,
                   "tau_offset": round(tau_value, 4),
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
