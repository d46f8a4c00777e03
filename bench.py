"""Benchmark: tree-masked prefill attention on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload c3] [--no-cpu-baseline]

One step is one ``dan_amd.attend`` call (one fused kernel launch) over the
whole packed batch, inputs resident in HBM. The default workload is the
Llama-3-8B attention shape (32 q / 8 kv heads, head_dim 128, bf16) at the
8192-token serving budget with a shared 1024-token prefix-cache block
(seed 0: 5 requests, 45 branches).

Prints one JSON line:
  value         useful TFLOP/s: 4 * D * H * (visible query-key pairs) / step time
  tokens_per_s  packed tokens per second
  roofline      the fused kernel against the bf16 dense matrix-core peak, from
                HIP events around a block of back-to-back launches on the
                launch stream (an event between two launches idles the GPU)
  cpu_baseline  the masked CPU path (oracle restatement of the reference's
                dense path, fp32, torch SDPA) on this host's cores
"""
import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = {"bf16": 2516.6, "fp16": 2516.6, "fp32": 2516.6, "fp8": 5033.2}  # dense matrix-core peaks
HBM_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def useful_flops(w):
    from dan_amd.workloads import useful_pairs

    return 4 * w.q.shape[2] * w.q.shape[0] * useful_pairs(w.segments)


def algorithmic_bytes(w):
    """Q + K + V read once, O written once (bf16 for e4m3 inputs), plus each
    distinct past tensor once."""
    h, n, d = w.q.shape
    hkv = w.k.shape[0]
    es = w.q.element_size()
    es_out = 2 if w.q.dtype == torch.float8_e4m3fn else es
    total = (n * h * d + 2 * n * hkv * d) * es + n * h * d * es_out
    seen = set()
    for s in w.segments:
        if s.past and id(s.past) not in seen:
            seen.add(id(s.past))
            pk, pv = s.past[w.layer][:2]
            total += pk.numel() * pk.element_size() + pv.numel() * pv.element_size()
    return total


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_cpus():
    """CPUs this process may run on: its affinity mask, capped by the cgroup's
    CPU quota when one is set (a container's share of a larger machine).
    Returns (cpus, affinity, quota or None)."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = max(1, math.ceil(int(q) / int(period)))
    except (OSError, ValueError):
        pass
    return (min(affinity, quota) if quota else affinity), affinity, quota


def cpu_baseline(name, seed, flops, n_tokens):
    """Oracle (reference dense path restated) on the host: 1 warm-up, median of 3,
    with one torch thread per CPU the process may use."""
    from dan_amd import workloads
    from oracle.tree_attention import attend_dense

    threads, affinity, quota = host_cpus()
    torch.set_num_threads(threads)
    if name == "c5":  # e4m3 inputs: the CPU path runs on config 3's originals (same useful FLOPs)
        name = "c3"
    w = {**workloads.CONFIGS, **workloads.EXTRA}[name](seed, device="cpu")
    attend_dense(w.q, w.k, w.v, w.segments, w.layer)
    times = []
    for _ in range(3):
        t = time.perf_counter()
        attend_dense(w.q, w.k, w.v, w.segments, w.layer)
        times.append(time.perf_counter() - t)
    t = statistics.median(times)
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"full {name} seed {seed} workload ({n_tokens} packed tokens), fp32 torch SDPA per segment, "
                      f"1 warm-up then median of 3 runs ({t:.3f} s); {threads} threads = the process's CPUs "
                      f"(affinity {affinity}, cgroup quota {quota if quota else 'none'}); CPU: {cpu_model()}",
            "seconds": round(t, 4), "tokens_per_s": round(n_tokens / t, 1)}


def forward_layers(w, layers, forwards):
    """A model forward's attention: a fresh Batch (so the tile plan is built
    again) whose prefix entry holds one (k, v) per layer, then ``layers``
    attend calls (each layer's prefix table built on its first call). Returns
    ms per forward (median over ``forwards``, after one untimed forward)."""
    from dataclasses import replace

    from dan_amd.attention import Batch, attend

    kw = w.attend_kwargs
    shared = {}
    times = []
    for f in range(forwards + 1):
        segs = Batch()
        for s in w.segments:
            past = None
            if s.past:
                if id(s.past) not in shared:
                    entry = s.past[w.layer]
                    # one prefix entry per layer: fresh tensors of the same shape (and scales)
                    shared[id(s.past)] = {l: tuple(t.clone() for t in entry) for l in range(layers)}
                past = shared[id(s.past)]
            segs.append(replace(s, past=past, saved={}, _mask=None))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for layer in range(layers):
            attend(w.q, w.k, w.v, segs, layer, **kw)
        torch.cuda.synchronize()
        if f:
            times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


def copy_calibration(mib, steps):
    """A plain copy of known size: FETCH_SIZE and WRITE_SIZE of its dispatches
    give the counters' scale (read bytes = written bytes = mib MiB each)."""
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "copies": steps}), flush=True)


FRONT_SHAPES = {
    # name: (tokens, q heads, kv heads, head_dim, rotary dims, q/k norm)
    "c3": (8192, 32, 8, 128, 128, None),        # Llama-3-8B: full RoPE, no q/k norm
    "c4": (8192, 32, 8, 128, 128, "rms"),       # Qwen3-4B-style: per-head RMSNorm on q and k
}


def bench_front(args):
    """The attention front end (dan_amd.front.qkv_front) on the named shape:
    one step = one launch over q and k of a fused projection output,
    HBM-bound; the metric is algorithmic GB/s against 8 TB/s."""
    from dan_amd.front import qkv_front
    n, h, hkv, d, r, norm = FRONT_SHAPES[args.workload]
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(args.seed)
    qkv = torch.randn(n, (h + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(dev)
    qx, kx, vx = qkv.split([h * d, hkv * d, hkv * d], dim=-1)
    q, k, v = qx.reshape(n, h, d), kx.reshape(n, hkv, d), vx.reshape(n, hkv, d)
    pos = torch.arange(n, dtype=torch.float32)
    inv = 1.0 / (500000.0 ** (torch.arange(0, r, 2, dtype=torch.float64) / r)).float()
    ang = torch.cat((pos[:, None] * inv[None, :],) * 2, dim=-1)
    cos, sin = ang.cos().to(torch.bfloat16).to(dev), ang.sin().to(torch.bfloat16).to(dev)
    w = torch.ones(d, dtype=torch.bfloat16, device=dev)
    call = lambda: qkv_front(q, k, v, cos, sin, q_norm_weight=w, k_norm_weight=w, norm=norm)
    # Back-to-back launches with no host synchronization between the settle
    # calls, the warm-up and the timed block (an idle GPU drops its clock):
    # the block's two events give the average launch time; per-launch events
    # afterwards give the median.
    stream = torch.cuda.current_stream(dev)
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < args.settle_ms:
        for _ in range(10):
            call()
        stream.query()
    for _ in range(args.warmup):
        call()
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b0.record(stream)
    for _ in range(args.steps):
        call()
    b1.record(stream)
    torch.cuda.synchronize()
    k_avg = b0.elapsed_time(b1) / args.steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for e0, e1 in ev:
        e0.record(stream)
        call()
        e1.record(stream)
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in ev]
    nbytes = 2 * (n * h * d + n * hkv * d) * 2 + 2 * n * r * 2  # read q, k and cos, sin; write q, k
    gbps = nbytes / (k_avg * 1e-3) / 1e9
    print(json.dumps({
        "metric": "attention front end (q/k norm + RoPE + layout) algorithmic GB/s, 1 GPU",
        "value": round(gbps, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        # the block's GPU time per launch: the host enqueues far ahead of the GPU
        # during the settle calls, so its wall clock would count that backlog
        "ms_per_step": round(k_avg, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"front-{args.workload}: {n} tokens, {h}/{hkv} heads, head_dim {d}, rotary {r}, "
                               f"q/k norm {norm}", "seed": args.seed},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_GBPS, 4), "traffic": None, "kernel_ms_avg": round(k_avg, 4),
                     "kernel_ms_median": round(statistics.median(ms), 4), "algorithmic_mb": round(nbytes / 1e6, 2)},
        "cpu_baseline": None,
    }), flush=True)


LLAMA8B_LINEARS = (("qkv_proj", 6144, 4096), ("o_proj", 4096, 4096), ("gate_up_proj", 28672, 4096),
                   ("down_proj", 4096, 14336))  # (name, out_features, in_features) of one decoder layer


def _event_ms(fn, steps):
    """Average ms per call of ``steps`` back-to-back calls between two events
    (an event between two calls would idle the GPU for several us)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_fp8_linear(args):
    """One decoder layer's FP8 linears (dan_amd.quant.FP8Linear, rowwise) at
    Llama-3-8B shapes on 8192 tokens: activation quantization and the scaled
    e4m3 GEMM per linear, both this package's kernels. One step = the four
    linears' forwards on synthetic bf16 activations and random weights.
    The GEMM is timed on the tiled operands FP8Linear hands it (`gemm_ms`),
    on row-major operands (`rows_gemm_ms`), and hipBLASLt's GEMM
    (torch._scaled_mm, dan's call) on the same codes (`hipblaslt_gemm_ms`)."""
    from torch import nn

    from dan_amd.quant import FP8Linear, fp8_gemm, fp8_quantize

    dev = torch.device("cuda:0")
    m = 8192
    g = torch.Generator(device=dev).manual_seed(args.seed)
    layers, xs = [], []
    for name, n, k in LLAMA8B_LINEARS:
        lin = nn.Linear(k, n, bias=False, device=dev, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(n, k, device=dev, generator=g) * 0.02)
        layers.append(FP8Linear(lin, rowwise=True))
        xs.append(torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16))
    flops = sum(2 * m * n * k for _, n, k in LLAMA8B_LINEARS)

    def step():
        for f, x in zip(layers, xs):
            f(x)

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < args.settle_ms:
        step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t) / args.steps
    # parts, timed per launch on the stream
    quant_ms = [_event_ms(lambda x=x: fp8_quantize(x, tiled=True), args.steps) for x in xs]
    qs = [fp8_quantize(x) for x in xs]  # row-major codes (hipBLASLt's and the row-major GEMM's operand)
    qt = [fp8_quantize(x, tiled=True) for x in xs]
    gemm_ms = [_event_ms(lambda f=f, q=q: fp8_gemm(q[0], q[1], f.tiled_weight(), f.weight_scale, None, torch.bfloat16),
                         args.steps) for f, q in zip(layers, qt)]
    rows_ms = [_event_ms(lambda f=f, q=q: fp8_gemm(q[0], q[1], f.weight, f.weight_scale, None, torch.bfloat16),
                         args.steps) for f, q in zip(layers, qs)]
    for f, q in zip(layers, qs):  # hipBLASLt picks its kernel on a shape's first call
        torch._scaled_mm(q[0], f.weight.t(), scale_a=q[1], scale_b=f.weight_scale, out_dtype=torch.bfloat16)
    lib_ms = [_event_ms(lambda f=f, q=q: torch._scaled_mm(q[0], f.weight.t(), scale_a=q[1], scale_b=f.weight_scale,
                                                          out_dtype=torch.bfloat16), args.steps)
              for f, q in zip(layers, qs)]

    def eager_quant(x):  # dan/fused.py:85-91 as eager torch ops on this GPU
        xf = x.float()
        scale = xf.abs().amax(dim=-1, keepdim=True).clamp(min=1e-12) / 448.0
        return (xf / scale).to(torch.float8_e4m3fn), scale

    eager_ms = [_event_ms(lambda x=x: eager_quant(x), args.steps) for x in xs]
    qbytes = [m * k * 2 + m * k + m * 4 for _, _, k in LLAMA8B_LINEARS]
    gemm_tf = flops / (sum(gemm_ms) * 1e-3) / 1e12
    lib_tf = flops / (sum(lib_ms) * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import quant as OQ
        torch.set_num_threads(min(16, os.cpu_count() or 1))
        rows = 64
        sample_flops = sum(2 * rows * n * k for _, n, k in LLAMA8B_LINEARS)
        cx = [torch.randn(rows, k).to(torch.bfloat16) for _, _, k in LLAMA8B_LINEARS]
        cw = [(f.weight.cpu(), f.weight_scale.cpu()) for f in layers]
        tc = time.perf_counter()
        for x, (wq, ws) in zip(cx, cw):
            xq, sx = OQ.fp8_quantize(x, True)
            OQ.fp8_linear(xq, sx, wq, ws)
        tc = time.perf_counter() - tc
        cpu = {"value": round(sample_flops / tc / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
               "kind": "port", "sample": f"{rows} tokens through the four linears with the oracle (fp32 quantize, "
                                         f"float64 GEMM): {tc:.2f} s; CPU: {cpu_model()}"}
    print(json.dumps({
        "metric": "FP8 decoder linears (Llama-3-8B layer, 8192 tokens) TFLOP/s, 1 GPU",
        "value": round(flops / wall / 1e12, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8", "data": "synthetic",
        "config": {"workload": "fp8-linears: Llama-3-8B qkv/o/gate_up/down at 8192 tokens, rowwise e4m3",
                   "seed": args.seed},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tf, 1), "peak": PEAK_TFLOPS["fp8"], "unit": "TFLOP/s",
                     "frac": round(gemm_tf / PEAK_TFLOPS["fp8"], 4), "traffic": None,
                     "gemm_ms": [round(x, 4) for x in gemm_ms],
                     "gemm_tflops": [round(2 * m * n * k / (t * 1e-3) / 1e12, 1)
                                     for (_, n, k), t in zip(LLAMA8B_LINEARS, gemm_ms)],
                     "rows_gemm_ms": [round(x, 4) for x in rows_ms],
                     "hipblaslt_gemm_ms": [round(x, 4) for x in lib_ms], "hipblaslt_frac": round(lib_tf / PEAK_TFLOPS["fp8"], 4),
                     "quant_ms": [round(x, 4) for x in quant_ms],
                     "quant_gbps": [round(b / (t * 1e-3) / 1e9, 1) for b, t in zip(qbytes, quant_ms)],
                     "quant_hbm_frac": round(sum(qbytes) / (sum(quant_ms) * 1e-3) / 1e9 / HBM_GBPS, 4),
                     "eager_quant_ms": [round(x, 4) for x in eager_ms]},
        "cpu_baseline": cpu,
    }), flush=True)


def bench_gdn(args):
    """The Gated DeltaNet recurrence of one layer over the c3 tree batch, as
    dan/models/qwen3_5.py:198-210 phases it: every trunk from its segment's
    state (the prefix cache's state for a segment with a past, else zeros),
    then every branch from its trunk's final state. Head shape: 16 key and
    16 value heads of 128 (a Qwen3.5-style DeltaNet layer); synthetic
    post-convolution q, k, v and gates. One step = the two phase calls."""
    from dan_amd import workloads
    from dan_amd.deltanet import delta_rule

    dev = torch.device("cuda:0")
    w = workloads.config3(args.seed, device="cpu")
    hk = hv = 16
    d = 128
    trunks = [(s.start, s.trunk) for s in w.segments]
    branches = [(a, b - a, i) for i, s in enumerate(w.segments) for a, b in s.branches]
    n = w.num_tokens
    g = torch.Generator(device=dev).manual_seed(args.seed)
    q = torch.randn(n, hk, d, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(n, hk, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(n, hv, d, device=dev, generator=g).to(torch.bfloat16)
    gate = -(torch.rand(n, hv, device=dev, generator=g) * 0.1)
    beta = torch.rand(n, hv, device=dev, generator=g)
    init = torch.randn(len(trunks), hv, d, d, device=dev, generator=g) * 0.05
    trow = torch.cat([torch.arange(a, a + t) for a, t in trunks]).to(dev)
    brow = torch.cat([torch.arange(a, a + m) for a, m, _ in branches]).to(dev)
    bseg = torch.tensor([i for _, _, i in branches], device=dev, dtype=torch.int32)  # the branch phase's state_index
    tl, bl = [t for _, t in trunks], [m for _, m, _ in branches]
    out = torch.empty(n, hv, d, dtype=torch.bfloat16, device=dev)

    def step():
        ot, ft = delta_rule(q[trow], k[trow], v[trow], gate[trow], beta[trow], tl, init)
        out[trow] = ot
        ob, _ = delta_rule(q[brow], k[brow], v[brow], gate[brow], beta[brow], bl, ft, state_index=bseg)
        out[brow] = ob

    t_settle = time.perf_counter()  # the clock settles under sustained steps (see --settle-ms)
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t) / args.steps
    ft = delta_rule(q[trow], k[trow], v[trow], gate[trow], beta[trow], tl, init)[1]
    tr_ms = _event_ms(lambda: delta_rule(q[trow], k[trow], v[trow], gate[trow], beta[trow], tl, init), args.steps)
    br_ms = _event_ms(lambda: delta_rule(q[brow], k[brow], v[brow], gate[brow], beta[brow], bl, ft, state_index=bseg),
                      args.steps)
    forms = {}  # each phase's delta rule alone (inputs gathered beforehand), in each form
    tin = [x[trow] for x in (q, k, v, gate, beta)]
    bin_ = [x[brow] for x in (q, k, v, gate, beta)]
    for form in ("token", "chunk"):
        forms[form] = {
            "trunk_phase_ms": round(_event_ms(lambda: delta_rule(*tin, tl, init, form=form), args.steps), 4),
            "branch_phase_ms": round(_event_ms(lambda: delta_rule(*bin_, bl, ft, form=form, state_index=bseg),
                                               args.steps), 4)}
    tokens = len(trow) + len(brow)
    flops = tokens * hv * 7 * d * d  # per token and head: decay, S^T k, the rank-1 write, S^T q
    layer = _gdn_layer_times(args, w, hk, hv, d, dev)
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import deltanet as OD
        torch.set_num_threads(min(16, os.cpu_count() or 1))
        ct = [x.cpu()[trow.cpu()] for x in (q, k, v, gate, beta)]
        cb = [x.cpu()[brow.cpu()] for x in (q, k, v, gate, beta)]
        init_c, bseg_c = init.cpu(), bseg.cpu()
        reps, tc = 0, time.perf_counter()
        while True:  # whole layer steps, both phases, until about 5 s of CPU work
            fc = OD.delta_rule(*ct, tl, init_c)[1]
            OD.delta_rule(*cb, bl, fc.index_select(0, bseg_c))
            reps += 1
            if time.perf_counter() - tc > 5.0:
                break
        tc = time.perf_counter() - tc
        cpu = {"value": round(reps * tokens / tc, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{reps} whole layer steps ({tokens} tokens x {hv} heads, trunk then branch phase) through "
                         f"the oracle's chunked form (the reference's delta_rule_torch restated, fp32): {tc:.2f} s; "
                         f"CPU: {cpu_model()}"}
    print(json.dumps({
        "metric": "Gated DeltaNet recurrence, one layer over the c3 tree batch, tokens/s, 1 GPU",
        "value": round(tokens / wall, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 state, bf16 io", "data": "synthetic",
        "config": {"workload": f"gdn-c3: {len(trunks)} trunks (longest {max(tl)}), {len(bl)} branches, {tokens} tokens, "
                               f"{hk}/{hv} heads, Dk = Dv = {d}", "seed": args.seed},
        "roofline": {"bound": "sequential in chunks of 64 tokens per run (the chunked form; a phase whose longest "
                              "run is under deltanet.CHUNK_MIN_RUN tokens goes token by token); fp32 arithmetic, on "
                              "bf16 MFMA with fp32 operands as bf16 pairs for bf16 inputs; peak: the fp32 MFMA rate",
                     "achieved": round(flops / wall / 1e12, 2),
                     "peak": 157.3, "unit": "TFLOP/s", "frac": round(flops / wall / 1e12 / 157.3, 4), "traffic": None,
                     "trunk_phase_ms": round(tr_ms, 4), "branch_phase_ms": round(br_ms, 4), "forms": forms,
                     "longest_run_tokens": max(tl), "us_per_token_longest_run": round(tr_ms * 1e3 / max(tl), 3)},
        "layer": layer,
        "cpu_baseline": cpu,
    }), flush=True)


def bench_gdn_forms(args):
    """Both delta rule forms on synthetic phases of R runs of L tokens (16/16
    heads, Dk = Dv = 128, bf16): the measurement behind deltanet.CHUNK_MIN_RUN.
    Prints one JSON line per (R, L) with each form's median ms per call."""
    from dan_amd.deltanet import delta_rule

    dev = torch.device("cuda:0")
    for r in (45, 200):
        for ln in (4, 8, 16, 24, 32, 48, 64, 96, 128, 256):
            n = r * ln
            g = torch.Generator(device=dev).manual_seed(args.seed)
            q = torch.randn(n, 16, 128, device=dev, generator=g).bfloat16()
            k = torch.randn(n, 16, 128, device=dev, generator=g).bfloat16()
            v = torch.randn(n, 16, 128, device=dev, generator=g).bfloat16()
            gate = -(torch.rand(n, 16, device=dev, generator=g) * 0.1)
            beta = torch.rand(n, 16, device=dev, generator=g)
            st = torch.randn(r, 16, 128, 128, device=dev, generator=g) * 0.05
            ms = {}
            for form in ("token", "chunk"):
                fn = lambda: delta_rule(q, k, v, gate, beta, [ln] * r, st, form=form)
                for _ in range(3):
                    fn()
                ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
                for e0, e1 in ev:
                    e0.record()
                    fn()
                    e1.record()
                torch.cuda.synchronize()
                ms[form] = round(statistics.median(e0.elapsed_time(e1) for e0, e1 in ev), 4)
            print(json.dumps({"runs": r, "run_tokens": ln, "token_ms": ms["token"], "chunk_ms": ms["chunk"]}),
                  flush=True)


def _gdn_layer_times(args, w, hk, hv, d, dev, hidden=2048, kernel=4):
    """The whole DeltaNet layer (dan_amd.deltanet.DeltaNet: bf16 projections,
    conv phase, delta rule, gated norm, output projection) over the same tree
    with random weights, its layout built once per forward as dan shares it
    across layers; and the conv phase kernel alone on the trunk phase, with
    its algorithmic bytes (conv rows in and out, gate inputs and outputs)."""
    import dataclasses
    from types import SimpleNamespace

    from dan_amd.attention import Batch
    from dan_amd import _native
    from dan_amd.deltanet import DeltaNet, RecurrentLayout, conv_phase_args

    cfg = SimpleNamespace(linear_num_key_heads=hk, linear_num_value_heads=hv, linear_key_head_dim=d,
                          linear_value_head_dim=d, linear_conv_kernel_dim=kernel, hidden_size=hidden,
                          rms_norm_eps=1e-6)
    torch.manual_seed(args.seed)
    m = DeltaNet(cfg, 0).to(dev, torch.bfloat16)
    c = m.conv_dim
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    segs = Batch(dataclasses.replace(
        s, past={0: (torch.randn(kernel - 1, c, device=dev, generator=g).to(torch.bfloat16),
                     torch.randn(hv, d, d, device=dev, generator=g) * 0.05)} if s.past else None,
        saved={}, _mask=None) for s in w.segments)
    n = w.num_tokens
    x = torch.randn(n, hidden, device=dev, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        for _ in range(args.warmup):
            m(x, segs)
        layer_ms = _event_ms(lambda: m(x, segs), args.steps)
        qkv = torch.randn(n, c, device=dev, generator=g).to(torch.bfloat16)
        ba = torch.randn(n, 2 * hv, device=dev, generator=g).to(torch.bfloat16)
        hist = torch.cat([segs[i].past[0][0] for i in segs.recurrent.past_segments]) if segs.recurrent.past_segments else None
        ph = segs.recurrent.trunk1
        # The phase's arguments built once and the library called directly, so the
        # timing is the launches' (the Python wrapper's per-call set-up costs about as
        # much as the kernels).
        cx, _, keep = conv_phase_args(qkv, hist, ph, m.conv1d.weight, ba[:, :hv], ba[:, hv:], m.A_log, m.dt_bias)
        stream = torch.cuda.current_stream(dev).cuda_stream
        fn = lambda: _native.gdn_conv(cx, stream)
        fn()
        conv_ms = _event_ms(fn, args.steps)
    t = len(ph.rows)
    conv_bytes = (t * c * 2) * 2 + t * hv * (2 * 2 + 4 * 2)
    return {"hidden": hidden, "conv_dim": c, "kernel": kernel, "layer_ms": round(layer_ms, 4),
            "layer_tokens_per_s": round(n / layer_ms * 1e3, 1), "conv_phase_rows": t,
            "conv_phase_ms": round(conv_ms, 4), "conv_phase_gbps_algorithmic": round(conv_bytes / conv_ms / 1e6, 1)}


def bench_plan(args):
    """Per-forward tile planning: the host planner (numpy tables, schedule
    and uploads) against the device planner (O(segments) host part, one
    upload, one planner launch), each until its tables are on the GPU (a
    synchronize ends every step). The attention call itself is not timed."""
    from dan_amd import _native, workloads
    from dan_amd.attention import _num_cus
    from dan_amd.plan import TilePlan

    lib = _native.load()
    dev = torch.device("cuda:0")
    w = {**workloads.CONFIGS, **workloads.EXTRA}[args.workload](args.seed, device=dev)
    h, hkv = w.q.shape[0], w.k.shape[0]
    tile_q = _native.tile_q(h, hkv, w.q.shape[2], lib=lib)
    groups, cus = _native.head_groups(h, hkv, lib), _num_cus(dev)

    def host():
        TilePlan.build(w.segments, w.num_tokens, tile_q, dev).schedule(groups, cus)

    def device():
        TilePlan.build_device(w.segments, w.num_tokens, tile_q, dev, groups, cus)

    res = {}
    for name, fn in (("host", host), ("device", device)):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        wall, gpu = [], []
        for _ in range(args.steps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t = time.perf_counter()
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            wall.append(time.perf_counter() - t)
            gpu.append(e0.elapsed_time(e1))
        res[name] = (statistics.median(wall) * 1e6, statistics.median(gpu) * 1e3)
    print(json.dumps({
        "metric": "tile planning latency per forward (tables on the GPU), 1 GPU", "value": round(res["device"][0], 1),
        "unit": "us", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(res["device"][0] / 1e3, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "int32", "data": "synthetic",
        "config": {"workload": f"planner-{args.workload}: {len(w.segments)} segments, {w.num_tokens} tokens, "
                               f"tile_q {tile_q}, {groups} head groups, {cus} CUs", "seed": args.seed},
        "host_planner_us": round(res["host"][0], 1), "device_planner_us": round(res["device"][0], 1),
        "device_stream_us": round(res["device"][1], 1), "speedup": round(res["host"][0] / res["device"][0], 2),
        "roofline": None, "cpu_baseline": None,
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c3", choices=["c1", "c2", "c3", "c4", "c5", "q35"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--settle-ms", type=float, default=2000.0,
                    help="untimed calls of the same workload before the warm-up steps, until this much wall "
                         "time has passed: under sustained load the GPU's clock keeps ramping for about 2 s "
                         "(c3: 0.327 ms per call after 0.3 s, 0.281 ms after 2 s)")
    ap.add_argument("--forward-layers", type=int, default=32,
                    help="also time a model forward of this many attention layers (fresh plan, per-layer prefix "
                         "tables; 0 skips it)")
    ap.add_argument("--front", action="store_true",
                    help="measure the attention front end (q/k norm + RoPE + layout) on --workload c3 or c4 "
                         "instead of the attention")
    ap.add_argument("--fp8-linear", action="store_true",
                    help="measure one Llama-3-8B decoder layer's FP8 linears (quantize + hipBLASLt GEMM) at 8192 tokens")
    ap.add_argument("--gdn", action="store_true",
                    help="measure the Gated DeltaNet recurrence of one layer over the c3 tree batch")
    ap.add_argument("--gdn-forms", action="store_true",
                    help="time both delta rule forms on phases of R runs of L tokens (the form threshold)")
    ap.add_argument("--plan", action="store_true",
                    help="measure per-forward tile planning (host planner against the device planner) on --workload")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="instead of attention, run --steps plain device copies of this many MiB (the calibration "
                         "kernel for the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the tree-attention path runs on a single device "
              "(see DESIGN.md for how it would shard); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    if args.copy_mib:
        copy_calibration(args.copy_mib, args.steps)
        return
    if args.plan:
        bench_plan(args)
        return
    if args.fp8_linear:
        bench_fp8_linear(args)
        return
    if args.gdn:
        bench_gdn(args)
        return
    if args.gdn_forms:
        bench_gdn_forms(args)
        return
    if args.front:
        if args.workload not in FRONT_SHAPES:
            print(f"--front measures {list(FRONT_SHAPES)}", file=sys.stderr)
            sys.exit(2)
        bench_front(args)
        return

    from dan_amd import _native, workloads
    from dan_amd.attention import attend

    _native.load()
    dev = torch.device("cuda:0")
    w = {**workloads.CONFIGS, **workloads.EXTRA}[args.workload](args.seed, device=dev)
    flops = useful_flops(w)
    nbytes = algorithmic_bytes(w)
    n = w.num_tokens
    dtype = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32",
             torch.float8_e4m3fn: "fp8"}[w.q.dtype]
    kw = w.attend_kwargs

    out = None
    settle_calls = 0
    t_settle = time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for _ in range(10):
            attend(w.q, w.k, w.v, w.segments, w.layer, **kw)
        torch.cuda.synchronize()
        settle_calls += 10
    # Nothing may idle the GPU between the settle and the timed steps: a pause
    # of a few milliseconds (a host-side check, a sleep) sends the clock into
    # a swing that costs the next ~20 ms of calls up to 30 % (c3: 0.281 ms per
    # call without a pause, 0.320 after a 5 ms sleep, 0.336 after a finiteness
    # check of the output). The outputs are checked after the timed region.
    # The timed steps run back to back with nothing else in the stream: an
    # event recorded between two calls idles the GPU for ~10 us at each one
    # (c3: 266 us per call with an event pair around every call against 256 us
    # without, in the kernel trace), so the timed block has one event at each
    # end, and per-call events come in a separate pass afterwards.
    stream = torch.cuda.current_stream(dev)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(args.warmup):
        out = attend(w.q, w.k, w.v, w.segments, w.layer, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    b0.record(stream)
    for i in range(args.steps):
        out = attend(w.q, w.k, w.v, w.segments, w.layer, **kw)
    b1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    call_block_ms = b0.elapsed_time(b1) / args.steps
    for i in range(args.steps):
        starts[i].record(stream)
        attend(w.q, w.k, w.v, w.segments, w.layer, **kw)
        ends[i].record(stream)
    torch.cuda.synchronize()
    call_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]

    # The attention launch alone (the dominant kernel; the V^T copy before it
    # is timed by difference), on the same stream, reading the copy one
    # PHASE_PACK call left in a workspace of its own: a block of back-to-back
    # launches between two events (the average), then one event pair per
    # launch (the median).
    from dan_amd.attention import _attend_fused, workspace_bytes
    fp8 = (kw["q_scale"], kw["k_scale"], kw["v_scale"]) if kw else None
    ws = torch.empty(workspace_bytes(w.q, w.k, w.segments), dtype=torch.uint8, device=dev)
    attend_only = lambda: _attend_fused(w.q, w.k, w.v, w.segments, w.layer, None, fp8, phases=_native.PHASE_ATTEND,
                                        workspace=ws)
    _attend_fused(w.q, w.k, w.v, w.segments, w.layer, None, fp8, phases=_native.PHASE_PACK, workspace=ws)
    b0.record(stream)
    for i in range(args.steps):
        attend_only()
    b1.record(stream)
    for i in range(args.steps):
        starts[i].record(stream)
        attend_only()
        ends[i].record(stream)
    torch.cuda.synchronize()
    kernel_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    if out is not None and not torch.isfinite(out).all():  # the last timed call's output
        raise RuntimeError("non-finite output")
    k_avg = b0.elapsed_time(b1) / args.steps
    k_med = statistics.median(kernel_ms)

    achieved = flops / (k_avg * 1e-3) / 1e12
    peak = PEAK_TFLOPS[dtype]
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get(f"{args.workload}_seed{args.seed}", {}).get("bytes_per_launch")

    line = {
        "metric": "tree-masked prefill attn TFLOP/s (useful) + packed tok/s, 8B shape, 1 GPU",
        "value": round(flops / (ms_step * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "tokens_per_s": round(n / (ms_step * 1e-3), 1),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_calls": settle_calls,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: " + ({**workloads.CONFIGS, **workloads.EXTRA}[args.workload].__doc__ or "").split(";")[0]
                   .strip().replace("\n", " "),
                   "seed": args.seed, "packed_tokens": n, "heads": f"{w.q.shape[0]}/{w.k.shape[0]}",
                   "head_dim": w.q.shape[2],
                   **{k: v for k, v in w.meta.items() if k != "packed_tokens" and not isinstance(v, torch.Tensor)},
                   "useful_gflop": round(flops / 1e9, 3), "algorithmic_mb": round(nbytes / 1e6, 2)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4), "traffic": traffic,
                     "kernel": "tree_attn_kernel (the attention launch; the fp16 V^T copy before it is in "
                               "call_ms_avg)",
                     "kernel_ms_avg": round(k_avg, 4), "kernel_ms_median": round(k_med, 4),
                     "kernel_timing": "kernel_ms_avg: a block of back-to-back launches between two events; "
                                      "kernel_ms_median and call_ms_median: one event pair per launch or call",
                     "call_ms_avg": round(call_block_ms, 4), "call_ms_median": round(statistics.median(call_ms), 4),
                     "hbm_gbps_algorithmic": round(nbytes / (k_avg * 1e-3) / 1e9, 1),
                     "hbm_frac_algorithmic": round(nbytes / (k_avg * 1e-3) / 1e9 / HBM_GBPS, 4),
                     "bf16_peak_frac": round(achieved / PEAK_TFLOPS["bf16"], 4)},
        "cpu_baseline": None,
    }
    if args.forward_layers:
        fwd_ms = forward_layers(w, args.forward_layers, 5)
        line["forward"] = {"layers": args.forward_layers, "ms": round(fwd_ms, 4),
                           "ms_per_layer": round(fwd_ms / args.forward_layers, 4),
                           "tflops": round(flops * args.forward_layers / (fwd_ms * 1e-3) / 1e12, 3),
                           "note": "wall time of one model forward's attention layers: a fresh Batch (tile plan "
                                   "rebuilt), one prefix entry per layer (each layer's table built on first use), "
                                   "then the attend calls; median of 5 forwards"}
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.workload, args.seed, flops, n)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
