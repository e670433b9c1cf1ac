#!/usr/bin/env python3
"""Benchmark of the INT4 KV-cache data plane on one MI355X.

Headline ("config 2"): one decode step of paged
attention over INT4 KV pages — batch 16, 32 heads, head_dim 128, context
4096 per sequence, 16-token pages (group-64 codes + fp16 scales), block
tables a seeded random permutation of the page pool, retain_ratio 1.0.
A "step" is one ``dynamic_sparse_attention`` call over the whole batch with
inputs resident in HBM. ``value`` = effective KV bytes (codes + fp16 scales,
285,212,672 B) / seconds per step, in GB/s.

The pool holds four disjoint page sets (1.14 GB) and steps rotate over
them, so a step never re-reads what earlier steps left in the 256 MB
last-level cache; the same launches rotating over two of the sets (570 MB)
are timed as a control and reported beside the headline. The JSON line also carries the roofline of the decode kernel (timed
with HIP events on the stream it runs on), a CPU baseline (the reference's
torch CPU path, restated in oracle/, on a bounded sample), and secondary
figures (prefill MFMA use, sparse and long-context decode with evict_tokens,
the KV-quant write path, and config 2's decode shape over an fp16 page pool).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 200] [--no-cpu] [--no-secondary]
       python bench.py --calibrate-copy | --decode-sweep
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "memopt-transformer-runtime_amd"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0
# The decode kernel instance the library launches for D=128 INT4 pages (default shape).
INT4_DECODE_KERNEL = "decode_int4_pages_kernel<128, 8, 1>"

CFG2 = dict(batch=16, heads=32, head_dim=128, ctx=4096, block=16, outlier_frac=0.005, outlier_mult=10.0, seed=0)


def effective_kv_bytes(batch, heads, head_dim, tokens):
    """Codes (D/2 bytes per token-head, K and V) + fp16 scales (D/64 per token-head, K and V)."""
    return 2 * batch * heads * tokens * (head_dim // 2 + 2 * (head_dim // 64))


def profile_traffic(name):
    """HBM bytes per launch recorded from rocprofv3 --pmc runs (profiles/), if present."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def setup_decode(torch, memopt_C, cfg, copies=2):
    """INT4 page pool with `copies` disjoint page sets for config 2."""
    B, H, D, ctx, bs = cfg["batch"], cfg["heads"], cfg["head_dim"], cfg["ctx"], cfg["block"]
    nbps = ctx // bs
    nb = copies * B * nbps
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    dev = torch.device("cuda", 0)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(cfg["seed"])).to(torch.int32)
    tables = [perm[c * B * nbps:(c + 1) * B * nbps].reshape(B, nbps).to(dev) for c in range(copies)]
    g = torch.Generator(device=dev).manual_seed(cfg["seed"])
    for bt in tables:
        slots = (bt.long()[:, :, None] * bs + torch.arange(bs, device=dev)).reshape(-1).to(torch.int32)
        for b0 in range(0, B, 4):
            n = min(4, B - b0) * ctx
            kv = []
            for _ in range(2):
                x = torch.randn(n, H, D, device=dev, generator=g)
                m = torch.rand(n, H, D, device=dev, generator=g) < cfg["outlier_frac"]
                kv.append(torch.where(m, x * cfg["outlier_mult"], x).half())
            memopt_C.write_cache(kv[0], kv[1], bt, slots[b0 * ctx:b0 * ctx + n].contiguous())
            del kv
    q = torch.randn(B, 1, H, D, device=dev, generator=g).half()
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    kc, vc = memopt_C.get_pool_tensors()
    calls = [memopt_C.PreparedAttention(q, kc, vc, bt, cl, ctx, ctx) for bt in tables]
    torch.cuda.synchronize()
    return calls, tables, q, cl


SETTLE_MS = 40.0


def settle(torch, fn, settle_ms=SETTLE_MS):
    """Runs `fn` (one launch or call per invocation) untimed until it has kept
    the GPU busy for `settle_ms` of GPU time (HIP events, checked every 50
    calls). Returns (host ms per call, GPU ms per call) over the settle.
    On MI355X the first 20-40 ms of a sustained phase run 5-15 % slower than
    the rest while the GPU's clocks adjust to it (config 5 decode: 405-416 us
    per launch over the first 100, then 357 us; config 2: 55 us, then
    47.5 us), and an idle GPU (a spin kernel holding the stream for 8 ms)
    loses that state again, so every figure here is taken right after such a
    settle, with the GPU kept busy in between: the sustained rate a serving
    loop sees."""
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    t0, n = time.perf_counter(), 0
    while True:
        for _ in range(50):
            fn()
        n += 50
        host_ms = (time.perf_counter() - t0) * 1e3 / n
        e1.record(stream)
        e1.synchronize()
        gpu_ms = e0.elapsed_time(e1) / n
        if gpu_ms * n >= settle_ms:
            return host_ms, gpu_ms


_BLOCK = {}


def fill(torch, fn, steps, warmup, host_ms, gpu_ms):
    """Untimed GPU work queued right before the timed calls, so that the host
    enqueues the `steps` timed calls while the GPU is still busy and they
    run back to back: `warmup` or more calls of `fn` when the host issues a
    call in well under its GPU time, otherwise (calls that cost the host more
    than the GPU) device copies covering 1.5x the host's enqueue time. Then
    a one-cycle spin kernel, a marker that puts the timed dispatches right
    after it in a kernel trace (the GPU idles a few microseconds, not the
    milliseconds a spin that holds the stream costs)."""
    if host_ms <= 0.7 * gpu_ms:
        for _ in range(max(warmup, int(steps * host_ms / (gpu_ms - host_ms)) + 2)):
            fn()
    else:
        for _ in range(warmup):
            fn()
        dev = torch.cuda.current_device()
        if dev not in _BLOCK:
            _BLOCK[dev] = (torch.empty(256 << 20, dtype=torch.uint8, device="cuda"),
                           torch.empty(256 << 20, dtype=torch.uint8, device="cuda"))
        src, dst = _BLOCK[dev]
        for _ in range(int(1.5 * steps * host_ms / 0.045) + 2):  # a 256 MiB copy takes ~45 us
            dst.copy_(src)
    torch.cuda._sleep(1)


def time_steps(torch, fn_list, steps, warmup, settle_ms=SETTLE_MS):
    """Returns (ms per step, host wall ms per step).

    After a settle of `settle_ms` of the same launches (see settle()) and
    the untimed fill (see fill(); it includes the `warmup` steps), `steps`
    launches run back to back on the current stream between two HIP events
    recorded on that stream, so the per-step time is the kernel's average
    duration (plus sub-microsecond dispatch gaps); it matches the AverageNs
    of `rocprofv3 --kernel-trace --stats` over the same dispatches.
    """
    stream = torch.cuda.current_stream()
    it = iter(range(1 << 62))
    nxt = lambda: fn_list[next(it) % len(fn_list)]()  # noqa: E731
    host_ms, gpu_ms = settle(torch, nxt, settle_ms)
    fill(torch, nxt, steps, warmup, host_ms, gpu_ms)
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    t_start.record(stream)
    for i in range(steps):
        fn_list[i % len(fn_list)]()
    t_end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    return t_start.elapsed_time(t_end) / steps, wall_ms


def cpu_model():
    """Host CPU model name from /proc/cpuinfo (None when unavailable)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline_config1(torch, O, reps=5):
    """BASELINE configs[0] on the host CPU, the reference's CPU route restated:
    group-64 quantize of K and V [64, 16, 8, 64] (src/csrc/quantization.cu
    semantics), dequantize, then single-query decode over the 1024 tokens
    through a random page permutation (gather, sinks U window, fp32 SDPA;
    src/memopt/triton_attention.py:473-550), 4 sinks, retain 1.0. Median of
    `reps` runs after one warm-up."""
    import numpy as np
    g = torch.Generator().manual_seed(0)
    k = O.outlier_normal(g, (64, 16, 8, 64), 0.01, 8.0)
    v = O.outlier_normal(g, (64, 16, 8, 64), 0.01, 8.0)
    q = torch.randn((1, 1, 8, 64), generator=g).half().numpy()
    bt = torch.randperm(64, generator=g).to(torch.int32).numpy()[None]
    cl = np.array([1024], np.int32)

    def step():
        kp, ks = O.quantize_int4(k)
        vp, vs = O.quantize_int4(v)
        return O.sdpa_fallback(q, O.dequantize_int4(kp, ks), O.dequantize_int4(vp, vs), bt, cl, 1024, 1024, 4)

    step()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    elems = 2 * k.size
    return {"workload": "BASELINE configs[0]: quantize K and V [64, 16, 8, 64], dequantize, decode over 1024 "
                        "tokens (random page permutation, 4 sinks), numpy/torch CPU",
            "ms_per_step": round(med * 1e3, 3), "quant_GB/s": round(elems * 2.5625 / med / 1e9, 4),
            "runs": reps}


def cpu_baseline_decode(torch, O, memopt_C, tables, q, cl, cfg, budget_s=15.0):
    """Reference CPU path (dequantize + gather + fp32 SDPA) on a bounded sample of config 2."""
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    bt = tables[0]
    nseq = 2
    pages = bt[:nseq].reshape(-1).long()
    # Copy only the sampled sequences' pages to host memory.
    sub = memopt_C.get_int4_pages()[pages].cpu()
    local_bt = torch.arange(pages.numel(), dtype=torch.int32).reshape(nseq, -1)
    qc, clc = q[:nseq].cpu(), cl[:nseq].cpu()
    ctx = cfg["ctx"]
    times = []
    O.decode_int4_torch(qc, sub, local_bt, clc, ctx, 0)  # warm-up
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 and time.perf_counter() < t_end:
        t0 = time.perf_counter()
        O.decode_int4_torch(qc, sub, local_bt, clc, ctx, 0)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    nbytes = effective_kv_bytes(nseq, cfg["heads"], cfg["head_dim"], ctx)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"{nseq} of {cfg['batch']} sequences of config 2 (dequantize + gather + fp32 SDPA, torch CPU), "
                      f"median of {len(times)} after 1 warm-up",
            "config1": cpu_baseline_config1(torch, O)}


def bench_fp16_decode(torch, memopt_C, cfg, steps=20):
    """Config 2's decode shape over an fp16 page pool (the reference's default
    cache format, 16-token pages), HBM GB/s on the K/V bytes streamed."""
    B, H, D, ctx, bs = cfg["batch"], cfg["heads"], cfg["head_dim"], cfg["ctx"], cfg["block"]
    nbps = ctx // bs
    nb = 2 * B * nbps  # two page sets, alternated, so repeats are not served by the last-level cache
    memopt_C.reset_pool()
    memopt_C.init_pool(nb, bs, H, D)
    dev = torch.device("cuda", 0)
    kc, vc = memopt_C.get_pool_tensors()
    g = torch.Generator(device=dev).manual_seed(cfg["seed"])
    for t in (kc, vc):
        for i in range(0, nb, 1024):
            t[i:i + 1024].copy_(torch.randn(t[i:i + 1024].shape, device=dev, generator=g))
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(cfg["seed"])).to(torch.int32)
    tables = [perm[c * B * nbps:(c + 1) * B * nbps].reshape(B, nbps).to(dev) for c in range(2)]
    q = torch.randn(B, 1, H, D, device=dev, generator=g).half()
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    calls = [memopt_C.PreparedAttention(q, kc, vc, bt, cl, ctx, ctx) for bt in tables]
    ms, _ = time_steps(torch, calls, steps, 5)
    nbytes = 2 * B * ctx * H * D * 2
    return {"workload": "config 2 decode shape over an fp16 page pool: batch 16, 32 heads, head_dim 128, "
                        "context 4096, 16-token pages, random-permutation block tables",
            "kernel": "decode_fp16_kernel<128, 4, 2>", "decode_ms": round(ms, 5), "bytes_streamed": nbytes,
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_fp16_write(torch, memopt_C, cfg, steps=20):
    """write_cache into the fp16 page pool bench_fp16_decode leaves: 4 x ctx
    tokens of config 2's K and V (2 x [16384, 32, 128]) into slots drawn at
    random from the pool (each token's H x D row lands on its own 8 KB), with
    validate_slots=False so the call is the scatter launch alone (the default
    check is a device min/max and one host read per call). GB/s on the bytes
    read and written."""
    H, D, ctx = cfg["heads"], cfg["head_dim"], cfg["ctx"]
    dev = torch.device("cuda", 0)
    T = 4 * ctx
    g = torch.Generator(device=dev).manual_seed(2)
    k = torch.randn(T, H, D, device=dev, generator=g).half()
    v = torch.randn(T, H, D, device=dev, generator=g).half()
    kc, _ = memopt_C.get_pool_tensors()
    nslots = kc.shape[0] * kc.shape[1]
    slots = torch.randperm(nslots, generator=torch.Generator().manual_seed(2))[:T].to(torch.int32).to(dev)
    bt = torch.zeros(1, 1, dtype=torch.int32, device=dev)
    ms, _ = time_steps(torch, [lambda: memopt_C.write_cache(k, v, bt, slots, validate_slots=False)], steps, 3)
    nbytes = 4 * T * H * D * 2
    return {"workload": "write_cache fp16 scatter, 2 x [16384, 32, 128] into random slots of an fp16 page pool",
            "kernel": "write_fp16_kernel", "kernel_ms": round(ms, 5), "bytes_moved": nbytes,
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_kv_quant(torch, memopt_C, cfg, steps=20):
    """Fused write + quantize of config 2's K and V into INT4 pages (write_cache), GB/s."""
    B, H, D, ctx, bs = cfg["batch"], cfg["heads"], cfg["head_dim"], cfg["ctx"], cfg["block"]
    dev = torch.device("cuda", 0)
    T = 4 * ctx  # 4 sequences per launch
    g = torch.Generator(device=dev).manual_seed(1)
    k = torch.randn(T, H, D, device=dev, generator=g).half()
    v = torch.randn(T, H, D, device=dev, generator=g).half()
    slots = torch.arange(T, dtype=torch.int32, device=dev)
    bt = torch.zeros(1, 1, dtype=torch.int32, device=dev)
    launch_ms, _ = time_steps(torch, [lambda: memopt_C.write_cache(k, v, bt, slots, validate_slots=False)], steps, 3)
    elems = 2 * T * H * D
    nbytes = elems * 2.53125
    return {"workload": "write_cache fused quantize, 2 x [16384, 32, 128] fp16 -> INT4 pages",
            "GB/s": round(nbytes / (launch_ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (launch_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "bytes_per_elem": 2.53125}


CFG4 = dict(batch=1, seq=16384, heads=32, head_dim=128, window=4096, sinks=4, block=16, std=0.5, seed=4)


def prefill_flops(seq, heads, head_dim, window, sinks):
    """4*D*H per (query, visible key) pair: QK^T and PV, 2 flops per MAC, causal
    StreamingLLM mask (key <= pos and (key < sinks or key > pos - window))."""
    total = 0
    for pos in range(seq):
        vis = min(pos + 1, window) + min(sinks, max(pos - window + 1, 0))
        total += vis
    return 4 * head_dim * heads * total


def bench_prefill(torch, memopt_C, cfg, steps=10, warmup=25):
    """Config 4: write_cache of 16384 tokens into INT4 pages, then causal paged
    attention (window 4096, 4 sinks) for all 16384 queries on the MFMA path.

    25 untimed calls (about 30 ms of MFMA load) come first: with 3, the timed
    calls of a fresh process ran about 5 % slower than the same calls timed
    again in that process, while the GPU's clock settled under the load."""
    S, H, D, bs = cfg["seq"], cfg["heads"], cfg["head_dim"], cfg["block"]
    dev = torch.device("cuda", 0)
    nb = S // bs
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(cfg["seed"])).to(torch.int32)
    bt = perm[None].to(dev)
    slots = (bt.long()[0, :, None] * bs + torch.arange(bs, device=dev)).reshape(-1).to(torch.int32)
    g = torch.Generator(device=dev).manual_seed(cfg["seed"])
    k = (torch.randn(S, H, D, device=dev, generator=g) * cfg["std"]).half()
    v = (torch.randn(S, H, D, device=dev, generator=g) * cfg["std"]).half()
    q = (torch.randn(1, S, H, D, device=dev, generator=g) * cfg["std"]).half()
    ctx = torch.tensor([S], dtype=torch.int32, device=dev)
    write_ms, _ = time_steps(torch, [lambda: memopt_C.write_cache(k, v, bt, slots, validate_slots=False)], steps,
                             warmup)
    kc, vc = memopt_C.get_key_pool(), memopt_C.get_value_pool()
    call = memopt_C.PreparedAttention(q, kc, vc, bt, ctx, S, cfg["window"], num_sink_tokens=cfg["sinks"],
                                      causal=True)
    launch_ms, _ = time_steps(torch, [call], steps, warmup)
    flops = prefill_flops(S, H, D, cfg["window"], cfg["sinks"])
    tflops = flops / (launch_ms * 1e-3) / 1e12
    return {"workload": "BASELINE configs[3]: B 1, seq 16384, 32 heads, head_dim 128, INT4 16-token pages, "
                        "causal window 4096 + 4 sinks, all 16384 queries",
            "kernel": "prefill_stage_kernel<128, true> (first head per XCD) + prefill_pipe_kernel<128, 4, true, true> "
                      "(stages the other heads)", "kernel_ms": round(launch_ms, 4),
            "flops": flops, "TFLOP/s": round(tflops, 1), "peak_TFLOP/s": MFMA_F16_PEAK_TFLOPS,
            "mfma_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "write_cache_ms": round(write_ms, 4)}


CFG3 = dict(batch=16, heads=32, head_dim=128, ctx=8192, block=16, retain=0.75, sinks=4, window=2048,
            outlier_frac=0.005, outlier_mult=10.0, seed=3)
CFG5 = dict(batch=4, heads=32, head_dim=128, ctx=131072, block=16, retain=0.75, sinks=4, spare_pages=4096,
            outlier_frac=0.01, outlier_mult=8.0, seed=5)


def fill_pages(torch, memopt_C, bt, cfg, gen):
    """write_cache of seeded K/V (N(0,1) with outliers) for every sequence of `bt`, one sequence at a time."""
    B, H, D, ctx, bs = bt.shape[0], cfg["heads"], cfg["head_dim"], cfg["ctx"], cfg["block"]
    dev = bt.device
    for b in range(B):
        slots = (bt[b].long()[:, None] * bs + torch.arange(bs, device=dev)).reshape(-1)[:ctx].to(torch.int32)
        kv = []
        for _ in range(2):
            x = torch.randn(ctx, H, D, device=dev, generator=gen)
            m = torch.rand(ctx, H, D, device=dev, generator=gen) < cfg["outlier_frac"]
            kv.append(torch.where(m, x * cfg["outlier_mult"], x).half())
            del x, m
        memopt_C.write_cache(kv[0], kv[1], bt, slots.contiguous())
        del kv


def bench_sparse_decode(torch, memopt_C, cfg, window, fifo_trace, copies=1, steps=20, warmup=3, control_copies=0):
    """evict_tokens (intended top-k, sinks kept) on LogNormal(0,1) scores, then
    INT4 decode over sinks U window. `copies` independent page sets (each
    filled and evicted on its own) are decoded in turn so that a working set
    smaller than the 256 MB last-level cache is not re-read from it. Returns
    the eviction time and the decode rate on the bytes of the pages the
    decode actually visits; with `control_copies`, also the rate when the
    steps rotate over only that many of the sets."""
    B, H, D, ctx, bs = cfg["batch"], cfg["heads"], cfg["head_dim"], cfg["ctx"], cfg["block"]
    dev = torch.device("cuda", 0)
    nbps = ctx // bs
    nb = copies * B * nbps + cfg.get("spare_pages", 0)
    memopt_C.init_pool(1, bs, H, D, kv_format="int4")  # identical parameters would keep the old free list
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    if fifo_trace:
        # allocate everything, free it in a seeded random order, then allocate
        # the sequences' pages from the FIFO: a fragmented block table
        got = [memopt_C.allocate_block() for _ in range(nb)]
        order = torch.randperm(nb, generator=torch.Generator().manual_seed(cfg["seed"])).tolist()
        for i in order:
            memopt_C.free_block(got[i])
        pages = torch.tensor([memopt_C.allocate_block() for _ in range(copies * B * nbps)], dtype=torch.int32)
    else:
        pages = torch.randperm(nb, generator=torch.Generator().manual_seed(cfg["seed"]))[:copies * B * nbps]
        pages = pages.to(torch.int32)
    gen = torch.Generator(device=dev).manual_seed(cfg["seed"])
    first_win = max(0, ctx - window) // bs
    vis = torch.zeros(nbps, dtype=torch.bool)
    vis[first_win:] = True
    vis[:(cfg["sinks"] + bs - 1) // bs] = True
    per_page = H * (2 * bs * (D // 2) + 2 * bs * 2 * (D // 64))
    calls, evict_ms, unlinked, nbytes = [], [], 0, 0
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    kc, vc = memopt_C.get_pool_tensors()
    for c in range(copies):
        bt = pages[c * B * nbps:(c + 1) * B * nbps].reshape(B, nbps).to(dev)
        fill_pages(torch, memopt_C, bt, cfg, gen)
        q = torch.randn(B, 1, H, D, device=dev, generator=gen).half()
        scores = torch.exp(torch.randn(B, H, ctx, device=dev, generator=gen))
        ibf = torch.zeros(nb, dtype=torch.int32, device=dev)
        memopt_C.evict_tokens(scores, bt, ibf, cfg["retain"], cfg["sinks"])
        if c == copies - 1:
            evict_ms.append(time_evict(torch, memopt_C, scores, bt, nb, cfg))
            evict_ms.append(time_evict_cold(torch, memopt_C, scores, bt, nb, cfg))
        unlinked += int((bt == -1).sum())
        nbytes += int(((bt.cpu() >= 0) & vis[None]).sum()) * per_page
        calls.append(memopt_C.PreparedAttention(q, kc, vc, bt, cl, ctx, window, num_sink_tokens=cfg["sinks"]))
        del scores
    nbytes //= copies  # bytes per step (copies are equal up to unlinked pages)
    ms, _ = time_steps(torch, calls, steps, warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"kernel": INT4_DECODE_KERNEL, "decode_ms": round(ms, 5), "bytes_streamed": nbytes,
           "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "evict_tokens_ms": round(evict_ms[0], 4), "evict_tokens_cold_ms": round(evict_ms[1], 4),
           "pages_unlinked": unlinked,
           "page_sets_rotated": copies,
           "block_tables": "seeded FIFO alloc/free trace" if fifo_trace else "seeded random permutation"}
    if control_copies:
        cms, _ = time_steps(torch, calls[:control_copies], steps, warmup)
        out["rotation_control"] = {"page_sets_rotated": control_copies, "decode_ms": round(cms, 5),
                                   "frac_of_hbm_peak": round(nbytes / (cms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def time_evict(torch, memopt_C, scores, bt, nb, cfg, reps=7):
    """Average time of evict_tokens on an already-evicted state: the same
    scores select the same tokens, so every call zeroes (again) the same rows
    and the work is that of the first call. Each call gets its own copy of the
    block tables (so unlinks do not accumulate) and a fresh vote counter, made
    before the timed region. The calls run back to back between two HIP
    events, after a settle and a fill (settle(), fill()) that keep the GPU
    busy while the host enqueues them, like the other figures of this bench;
    timing each call alone between its own events adds about 6 us of event
    overhead per call."""
    btcs = [bt.clone() for _ in range(reps + 1)]
    ibfs = [torch.zeros(nb, dtype=torch.int32, device=bt.device) for _ in range(reps + 1)]
    # settle and fill on one scratch copy (the same rows are zeroed again each call)
    scratch = lambda: memopt_C.evict_tokens(scores, btcs[reps], ibfs[reps], cfg["retain"], cfg["sinks"])  # noqa: E731
    host_ms, gpu_ms = settle(torch, scratch)
    fill(torch, scratch, reps, 1, host_ms, gpu_ms)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        memopt_C.evict_tokens(scores, btcs[i], ibfs[i], cfg["retain"], cfg["sinks"])
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def time_evict_cold(torch, memopt_C, scores, bt, nb, cfg, reps=7):
    """evict_tokens as time_evict() does it, but each call timed alone right
    after a 1 GiB device copy, so that no scale run, score or bitmask word of
    the previous call is still in the last-level cache (back-to-back calls
    find the scale runs the previous call rewrote there). Each call between
    its own HIP events, which adds about 1.5 us of event overhead per call."""
    btcs = [bt.clone() for _ in range(reps)]
    ibfs = [torch.zeros(nb, dtype=torch.int32, device=bt.device) for _ in range(reps)]
    src = torch.empty(1 << 30, dtype=torch.uint8, device=bt.device)
    dst = torch.empty_like(src)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for i in range(reps):
        dst.copy_(src)
        ev[i][0].record()
        memopt_C.evict_tokens(scores, btcs[i], ibfs[i], cfg["retain"], cfg["sinks"])
        ev[i][1].record()
    torch.cuda.synchronize()
    del src, dst
    return sum(a.elapsed_time(b) for a, b in ev) / reps


def bench_long_context_policy(torch, memopt_C, cfg, steps=20, warmup=3):
    """BASELINE configs[4] driven by the memory policy, as the reference
    intends (src/memopt/scheduler.py:338-384 -> the forward wrapper):
    a ThresholdPolicy with MemoryScheduler's rule and a near-zero high mark
    (SchedulerConfig(vram_high_threshold=eps, vram_low_threshold=0)) flips to
    use_int4=True, retain_ratio=0.75 on its first adjust_policy(); a
    PolicyForward step then converts the fp16 pool to INT4 pages, appends the
    step's token, decodes and evicts. The pool holds 4 x 131072 tokens from a
    fragmented FIFO free list (all pages allocated, then freed in a seeded
    order). Reported: the policy step's wall time, and the decode and
    evict_tokens kernels on the state it leaves."""
    sys.path.insert(0, os.path.join(ROOT, "memopt-transformer-runtime_amd"))
    from memopt_runtime import PagedKVCache, PolicyForward, ThresholdPolicy
    B, H, D, ctx, bs = cfg["batch"], cfg["heads"], cfg["head_dim"], cfg["ctx"], cfg["block"]
    nbps = ctx // bs
    nb = B * nbps + cfg["spare_pages"]
    dev = torch.device("cuda", 0)
    cache = PagedKVCache(nb, H, D, bs, kv_format="fp16")
    got = [memopt_C.allocate_block() for _ in range(nb)]
    for i in torch.randperm(nb, generator=torch.Generator().manual_seed(cfg["seed"])).tolist():
        memopt_C.free_block(got[i])
    seqs = list(range(B))
    for s in seqs:
        cache.add_sequence(s)
    g = torch.Generator(device=dev).manual_seed(cfg["seed"])

    def kv(T):
        out = []
        for _ in range(2):
            x = torch.randn(B, T, H, D, device=dev, generator=g)
            m = torch.rand(B, T, H, D, device=dev, generator=g) < cfg["outlier_frac"]
            out.append(torch.where(m, x * cfg["outlier_mult"], x).half())
            del x, m
        return out

    for t0 in range(0, ctx - 1, 8192):
        k, v = kv(min(8192, ctx - 1 - t0))
        cache.append(seqs, k, v)
        del k, v
    policy = ThresholdPolicy(vram_high_threshold=1e-9, vram_low_threshold=0.0, drop_retain_ratio=cfg["retain"])
    policy.adjust_policy()
    pf = PolicyForward(cache, policy, window_size=-1, num_sink_tokens=cfg["sinks"])
    q = torch.randn(B, 1, H, D, device=dev, generator=g).half()
    k1, v1 = kv(1)
    scores = torch.exp(torch.randn(B, H, ctx, device=dev, generator=g))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    pf.step(seqs, q, k1, v1, scores)
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3
    assert cache.kv_format == "int4" and pf.last_policy.retain_ratio == cfg["retain"]
    bt = cache.block_tables(seqs)
    cl = cache.context_lens(seqs)
    kc, vc = cache.key_value_pools()
    call = memopt_C.PreparedAttention(q, kc, vc, bt, cl, ctx, ctx, num_sink_tokens=cfg["sinks"])
    ms, _ = time_steps(torch, [call], steps, warmup)
    per_page = H * (2 * bs * (D // 2) + 2 * bs * 2 * (D // 64))
    linked = int((bt >= 0).sum())
    nbytes = linked * per_page
    gbs = nbytes / (ms * 1e-3) / 1e9
    evict_ms = time_evict(torch, memopt_C, scores, bt, nb, cfg)
    evict_cold_ms = time_evict_cold(torch, memopt_C, scores, bt, nb, cfg)
    return {"kernel": INT4_DECODE_KERNEL, "decode_ms": round(ms, 5), "bytes_streamed": nbytes,
            "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "evict_tokens_ms": round(evict_ms, 4), "evict_tokens_cold_ms": round(evict_cold_ms, 4),
            "pages_unlinked": B * nbps - linked,
            "policy": {"use_int4": pf.last_policy.use_int4, "retain_ratio": pf.last_policy.retain_ratio},
            "policy_step_ms": round(step_ms, 2),
            "policy_step": "fp16 -> INT4 pool conversion, 1-token append, decode, evict_tokens, free sweep",
            "block_tables": "fragmented FIFO free list (all pages allocated, freed in a seeded order)"}


def decode_page_sweep(torch, memopt_C, cfg=CFG3, copies=4, steps=20):
    """INT4 decode time against the pages each (b, h) visits, on config 3's
    shape (B 16, H 32, ctx 8192, random-permutation block tables, `copies`
    page sets rotated): windows of 1 to 256 pages (and 129 = config 3's
    2048-token window + the sink page). A least-squares line over the cases
    of 64 pages and more splits a launch into a fixed cost (intercept) and
    a streaming rate (slope)."""
    B, H, D, ctx, bs = cfg["batch"], cfg["heads"], cfg["head_dim"], cfg["ctx"], cfg["block"]
    dev = torch.device("cuda", 0)
    nbps = ctx // bs
    nb = copies * B * nbps
    memopt_C.init_pool(1, bs, H, D, kv_format="int4")
    memopt_C.init_pool(nb, bs, H, D, kv_format="int4")
    pages = torch.randperm(nb, generator=torch.Generator().manual_seed(cfg["seed"])).to(torch.int32)
    gen = torch.Generator(device=dev).manual_seed(cfg["seed"])
    kc, vc = memopt_C.get_pool_tensors()
    cl = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    bts, qs = [], []
    for c in range(copies):
        bt = pages[c * B * nbps:(c + 1) * B * nbps].reshape(B, nbps).to(dev)
        fill_pages(torch, memopt_C, bt, cfg, gen)
        bts.append(bt)
        qs.append(torch.randn(B, 1, H, D, device=dev, generator=gen).half())
    per_page = H * (2 * bs * (D // 2) + 2 * bs * 2 * (D // 64))
    cases = []
    for W, sinks in ((128, 0), (512, 0), (1024, 0), (2048, 0), (2048, 4), (4096, 0), (16, 0)):
        calls = [memopt_C.PreparedAttention(qs[c], kc, vc, bts[c], cl, ctx, W, num_sink_tokens=sinks)
                 for c in range(copies)]
        npages = W // bs + (1 if sinks else 0)
        ms, _ = time_steps(torch, calls, steps, 3)
        cases.append({"window": W, "sinks": sinks, "pages_per_bh": npages, "us": round(ms * 1e3, 3),
                      "frac_of_hbm_peak": round(B * npages * per_page / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    fit = [c for c in cases if c["pages_per_bh"] >= 64]
    n = len(fit)
    sx = sum(c["pages_per_bh"] for c in fit)
    sy = sum(c["us"] for c in fit)
    sxx = sum(c["pages_per_bh"] ** 2 for c in fit)
    sxy = sum(c["pages_per_bh"] * c["us"] for c in fit)
    slope = (n * sxy - sx * sy) / (n * sxx - sx * sx)
    icpt = (sy - slope * sx) / n
    return {"workload": "INT4 decode, B 16, H 32, D 128, ctx 8192, window swept", "cases": cases,
            "fit_fixed_us": round(icpt, 3), "fit_us_per_page": round(slope, 4),
            "fit_stream_frac_of_hbm_peak": round(B * per_page / (slope * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="skip secondary figures")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 5 plain 512 MiB device-to-device copies (scales rocprofv3 byte counters)")
    ap.add_argument("--decode-sweep", action="store_true",
                    help="only time INT4 decode against the pages per (b, h) (fixed cost and streaming rate)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the kernels run on one GPU's share of the "
              "work; sharding across GPUs is not built); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        n = 512 << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n, "launches": 5}))
        return
    import memopt_C  # noqa: E402  (fails loudly if the HIP library is missing)
    if args.decode_sweep:
        print(json.dumps(decode_page_sweep(torch, memopt_C)), flush=True)
        return

    cfg = CFG2
    calls, tables, q, cl = setup_decode(torch, memopt_C, cfg, copies=4)
    region_ms, wall_ms = time_steps(torch, calls, args.steps, args.warmup)
    # control: the same launches rotating over two of the four page sets
    control_ms, _ = time_steps(torch, calls[:2], args.steps, 20, settle_ms=10.0)
    nbytes = effective_kv_bytes(cfg["batch"], cfg["heads"], cfg["head_dim"], cfg["ctx"])
    value = nbytes / (region_ms * 1e-3) / 1e9
    achieved = value  # one decode launch per step
    line = {
        "metric": "INT4 paged decode-attn HBM GB/s (% peak); prefill MFMA util; KV-quant GB/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(region_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 codes, fp16 x fp16 -> fp32",
        "data": "synthetic (seeded N(0,1) K/V with 0.5% x10 outliers, quantized on device)",
        "config": {"workload": "BASELINE configs[1] decode: batch 16, 32 heads, head_dim 128, context 4096, "
                               "INT4 16-token pages (group 64, fp16 scales), random-permutation block tables, "
                               "retain_ratio 1.0",
                   "effective_kv_bytes": nbytes, "page_sets_rotated": len(calls),
                   "rotation_control": {"page_sets_rotated": 2, "ms_per_step": round(control_ms, 5),
                                        "frac_of_hbm_peak": round(nbytes / (control_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                                                  4)}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profile_traffic("decode_int4_config2_pmc.txt"),
                     "kernel": INT4_DECODE_KERNEL, "kernel_ms": round(region_ms, 5)},
    }
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O  # CPU baseline leg only
        line["cpu_baseline"] = cpu_baseline_decode(torch, O, memopt_C, tables, q, cl, cfg)
    if not args.no_secondary:  # re-initializes the pool: runs last
        sec = {"prefill": bench_prefill(torch, memopt_C, CFG4)}
        sec["sparse_decode_config3"] = dict(
            workload="BASELINE configs[2]: B 16, ctx 8192, evict_tokens r 0.75 + 4 sinks, decode window 2048",
            **bench_sparse_decode(torch, memopt_C, CFG3, CFG3["window"], fifo_trace=False, copies=6,
                                  control_copies=3))
        sec["long_context_config5"] = dict(
            workload="BASELINE configs[4]: B 4, ctx 131072, 32768 pages, scheduler-forced INT4 + retain 0.75, "
                     "4 sinks, full window, through PolicyForward",
            **bench_long_context_policy(torch, memopt_C, CFG5))
        sec["kv_quant"] = bench_kv_quant(torch, memopt_C, cfg)
        sec["fp16_pool_decode"] = bench_fp16_decode(torch, memopt_C, cfg)
        sec["fp16_write_cache"] = bench_fp16_write(torch, memopt_C, cfg)
        line["secondary"] = sec
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
