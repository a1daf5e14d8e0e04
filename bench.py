"""Benchmark of the fused 4-bit KV decode attention.

One step = one decode-attention call for a batch of 16 sequences at the
Qwen3-8B attention geometry (32 query / 8 KV heads, head_dim 128) over a
32768-token context: 32640 tokens in the 4-bit Format Q cache (K per channel
in groups of 32 tokens, V per token in groups of 32 channels, fp16
scale/zero) + a 128-token bf16 residual window.  Inputs are seeded Gaussian
bf16 values with 1% outlier K channels x10, quantized on the GPU by the pack
kernel and resident in HBM before timing; two independent caches (2 x 677 MB,
more than 2x the 256 MB MALL) alternate between steps so no step reads the
previous step's data from cache.

Prints one JSON line (the driver's contract) with the roofline of the main
kernel (HIP events on the launch stream around a batch of back-to-back
launches of that kernel, queued behind a short spin kernel so host launch
gaps are not counted) and the CPU baseline (the numpy oracle, one host
thread, on a bounded sample).

``--config c3`` (Quest page selection + page-sparse attention) and
``--config c4`` (RaBitQ search) print the same kind of line for the other
GPU configurations; the default is the headline configuration, C2.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

B, HQ, HKV, D, T, R = 16, 32, 8, 128, 32768, 128
NG = (T - R) // 32                      # 1020 quantized groups
BYTES_PER_TOKEN_Q = 160                 # K codes 64 + K meta 16 + V codes 64 + V meta 16
ALGO_BYTES = (B * HKV * NG * 32 * BYTES_PER_TOKEN_Q      # 4-bit cache
              + B * HKV * R * D * 2 * 2                  # bf16 residual K and V
              + B * HQ * D * 2 * 2)                      # q in, o out
HBM_PEAK_GBS = 8000.0
METRIC = "decode attn tokens/s + achieved HBM GB/s (% peak), 4-bit KV, 32k ctx, Qwen3-8B"


def make_cache(seed: int, device):
    from zoomkv_revision_amd import synthetic
    return synthetic.c2_cache(seed, B, HKV, NG, R, device)


def hbm_reference(caches, q, rounds: int = 6) -> dict:
    """GB/s of the C2 attention (algorithmic bytes) next to torch's device copy
    (read + write) and torch.sum (read) over the same byte volume, two
    alternating buffers each, in back-to-back batches of 20 launches."""
    import torch
    from zoomkv_revision_amd import kivi
    dev = q.device
    out = torch.empty(B, HQ, D, dtype=torch.bfloat16, device=dev)
    ws = kivi.attention_workspace(B, HQ, HKV, NG, R, 0, device=dev)
    srcs = [torch.ones(ALGO_BYTES // 4, dtype=torch.float32, device=dev) for _ in range(2)]
    dst = torch.empty_like(srcs[0])
    acc = torch.empty(1, dtype=torch.float32, device=dev)
    runs = {"c2_attention": (lambda i: kivi.kivi4_decode_attention(q, caches[i % 2], NG, R, out=out, workspace=ws), 1),
            "torch_copy_read_plus_write": (lambda i: dst.copy_(srcs[i % 2]), 2),
            "torch_sum_read": (lambda i: torch.sum(srcs[i % 2], dim=0, keepdim=True, out=acc), 1)}
    res = {k: [] for k in runs}
    for _ in range(rounds):
        for k, (fn, passes) in runs.items():
            res[k].append(passes * ALGO_BYTES / (kernel_batch_ms(fn, 20) * 1e-3) / 1e9)
    result = {"bytes": ALGO_BYTES, "unit": "GB/s", **{k: statistics.median(v) for k, v in res.items()}}
    # the same streams sustained: 240 back-to-back launches each, burst
    # (first 20) and settled (last 100) medians, ~1 s of idle between them
    for k, (fn, passes) in runs.items():
        torch.cuda._sleep(int(2e9))
        sus = sustained_ms(fn)
        result[k + "_sustained"] = {"burst_GBps": passes * ALGO_BYTES / (sus["burst_ms"] * 1e-3) / 1e9,
                                    "sustained_GBps": passes * ALGO_BYTES / (sus["sustained_ms"] * 1e-3) / 1e9}
    return result


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_cpu_threads(fn, budget_s: float = 10.0, max_calls: int = 20):
    """Median wall time of fn() on 1 thread and on every thread of the
    process's CPU share (torch.get_num_threads()), one warm-up call each;
    returns {threads: (median s, calls)}."""
    import torch
    n_all = torch.get_num_threads()
    res = {}
    for nt in (1, n_all):
        torch.set_num_threads(nt)
        fn()
        times = []
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(times) < 2:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if len(times) >= max_calls:
                break
        res[nt] = (statistics.median(times), len(times))
    torch.set_num_threads(n_all)
    return res


def cpu_baseline(cache, q, budget_s: float = 10.0, rows=(0,)):
    """The torch-CPU restatement of the C2 step (oracle/torch_cpu.py: 4-bit
    unpack + dequant, residual append, float32 SDPA with grouped heads) at
    the full per-sequence C2 shape (32 query / 8 KV heads, 32640 quantized +
    128 residual tokens), on a sample of the batch's sequences, timed with 1
    thread (as the reference cache sets, S:783-789) and with every thread of
    the process's CPU share."""
    import numpy as np
    import torch
    from oracle import torch_cpu
    r = list(rows)
    f16 = lambda t: t[r].cpu().view(torch.int16).numpy().view(np.uint16)
    prep = torch_cpu.prepare_c2(cache.k_codes[r].cpu().numpy(), f16(cache.k_meta), cache.v_codes[r].cpu().numpy(),
                                f16(cache.v_meta), cache.k_res[r, :, :R].float().cpu().numpy(),
                                cache.v_res[r, :, :R].float().cpu().numpy())
    q0 = q[r].float().cpu()
    n_all = torch.get_num_threads()
    res = {}
    for nt in (1, n_all):
        torch.set_num_threads(nt)
        torch_cpu.decode_attention(q0, prep, 1 / math.sqrt(D))            # warm-up
        times = []
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(times) < 2:
            t0 = time.perf_counter()
            torch_cpu.decode_attention(q0, prep, 1 / math.sqrt(D))
            times.append(time.perf_counter() - t0)
            if len(times) >= 20:
                break
        res[nt] = (statistics.median(times), len(times))
    torch.set_num_threads(n_all)
    (t1, n1), (tn, nn) = res[1], res[n_all]
    return {"value": len(r) / t1, "unit": "tokens/s", "cores": 1, "kind": "port",
            "all_cores": {"value": len(r) / tn, "cores": n_all},
            "cpu_model": cpu_model(), "host_logical_cpus": os.cpu_count(),
            "sample": f"torch-CPU restatement (oracle/torch_cpu.py) of the C2 step for {len(r)} of {B} "
                      f"sequences per call at the full per-sequence shape ({HQ} q / {HKV} KV heads, "
                      f"{NG * 32} + {R} tokens); median of {n1} calls ({t1:.2f} s) on 1 thread and "
                      f"{nn} calls ({tn:.2f} s) on {n_all} threads (torch.get_num_threads(), the "
                      f"process's CPU share; host {os.cpu_count()} logical CPUs, {cpu_model()})"}


def read_traffic(name: str = "kivi4_attn_c2_traffic.json"):
    """HBM bytes per launch from a committed counter summary under profiles/."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def timed_loop(step, steps: int, warmup: int) -> float:
    """Warm up, then time `steps` calls of step(i) bracketed by device
    synchronisation; returns wall-clock ms per step."""
    import torch
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def kernel_batch_ms(launch, n: int, host_us: float = 100.0) -> float:
    """Mean device time of the dominant kernel: n back-to-back launches between
    one pair of events on the launch stream.  A spin kernel ahead of the batch
    (host_us per launch) lets the host queue all n launches first, so host
    launch gaps are not counted (the figure rocprof's dispatch durations give)."""
    import torch
    launch(0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(2e3 * host_us) * n)  # ~2 GHz
    e0.record()
    for i in range(n):
        launch(i)
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / n


def sustained_ms(launch, n: int = 240, tail: int = 100, host_us: float = 40.0) -> dict:
    """Per-launch device times over n back-to-back launches (a HIP event
    between consecutive launches on the launch stream; a spin kernel ahead of
    the batch lets the host queue every launch first): the median of the
    first 20 (the burst the short timed regions see) and of the last `tail`
    (the settled rate under sustained load, after the power manager has
    lowered the clock)."""
    import torch
    launch(0)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    torch.cuda._sleep(int(2e3 * host_us) * n)  # ~2 GHz
    ev[0].record()
    for i in range(n):
        launch(i)
        ev[i + 1].record()
    ev[n].synchronize()
    d = [ev[i].elapsed_time(ev[i + 1]) for i in range(n)]
    return {"launches": n, "burst_ms": statistics.median(d[:20]), "sustained_ms": statistics.median(d[-tail:]),
            "max_ms": max(d)}


def run_c1(args):
    """C1: one layer, batch 1, 32 / 8 heads, 4096 tokens: KIVI 4-bit pack of the
    first 3968 tokens (124 groups), the 128-token bf16 residual window, then
    decode attention for one query token (inputs seeded on the CPU, seed 42)."""
    import torch
    from zoomkv_revision_amd import kivi, synthetic
    w = synthetic.c1_workload(42)
    nq, ng, res = w["n_quant"], w["n_groups"], w["res_len"]
    dev = torch.device("cuda:0")
    kd, vd, qd = w["k"].to(dev), w["v"].to(dev), w["q"].to(dev)
    cache = kivi.Kivi4Cache.allocate(1, 8, ng, res, device=dev)
    out = torch.empty(1, 32, 128, dtype=torch.bfloat16, device=dev)
    ws = kivi.attention_workspace(1, 32, 8, ng, res, 0, device=dev)

    # the range check records into a device word (no host synchronisation);
    # it is read once, after the timed steps
    kivi.kivi4_pack_status(dev)

    # the same buffers every call: the argument checks run once (PrefillPlan,
    # DecodeAttentionPlan), a step is two C-ABI calls
    prefill = kivi.PrefillPlan(kd, vd, cache, res)
    attend = kivi.DecodeAttentionPlan(qd, cache, ng, res, out=out, workspace=ws)

    def step(i):
        # one launch packs the 124 groups and copies the 128 residual rows
        prefill.run()
        attend.run()

    ms = timed_loop(step, args.steps, args.warmup)
    k_ms = kernel_batch_ms(lambda i: kivi.kivi4_prefill(kd, vd, cache, res), args.steps)
    kivi.check_kivi4_pack_range(dev)
    # bf16 K/V in (all 4096 tokens), Format Q records and the bf16 residual rows out
    pack_bytes = 8 * (nq + res) * 512 + 8 * nq * 160 + 8 * res * 512
    attn_bytes = 8 * nq * 160 + 8 * res * 512 + 2 * 32 * 128 * 2
    cpu = None if args.no_cpu else c1_cpu_baseline(w)
    return {
        "metric": "C1 one layer: KIVI 4-bit pack + decode attention, layer calls/s",
        "value": 1.0 / (ms * 1e-3), "unit": "layer calls/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 -> u4 codes + fp16 scale/zero; u4->fp16 attention (fp32 accumulate)",
        "data": "synthetic (seed 42, CPU generator)",
        "config": {"workload": "C1: pack 3968 tokens (124 groups) + 128-token bf16 residual + decode attention",
                   "batch": 1, "q_heads": 32, "kv_heads": 8, "head_dim": 128, "context": 4096,
                   "outlier_key_channels": 4, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": pack_bytes / (k_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": pack_bytes / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "traffic": read_traffic("c1_kivi4_pack_traffic.json"),
                     "kernel": "kivi4_pack_kernel (prefill: pack + residual rows)", "kernel_ms": k_ms,
                     "algorithmic_bytes": pack_bytes},
        "algorithmic_bytes_per_step": {"pack": pack_bytes, "attention": attn_bytes},
        "cpu_baseline": cpu,
    }


def c1_cpu_baseline(w, budget_s: float = 20.0):
    """numpy oracle of the whole C1 step (pack + attention) at full shape, timed
    with one thread and with every host core."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import kivi as okivi
    k, v, q = w["k"].float().numpy(), w["v"].float().numpy(), w["q"].float().numpy()
    nq, ng, res = w["n_quant"], w["n_groups"], w["res_len"]

    def once():
        c = okivi.quantize_kivi4(k[:, :, :nq], v[:, :, :nq])
        okivi.kivi4_decode_attention(q, c, ng, k[:, :, nq:], v[:, :, nq:], res, 1 / np.sqrt(128),
                                     dtype=np.float32)

    res_t = {}
    for threads in (1, os.cpu_count()):
        times = []
        with threadpool_limits(limits=threads):
            once()
            t_end = time.perf_counter() + budget_s / 2
            while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
                t0 = time.perf_counter()
                once()
                times.append(time.perf_counter() - t0)
        res_t[threads] = (statistics.median(times), len(times))
    t1, n1 = res_t[1]
    tn, nn = res_t[os.cpu_count()]
    return {"value": 1.0 / t1, "unit": "layer calls/s", "cores": 1, "kind": "port",
            "all_cores": {"value": 1.0 / tn, "cores": os.cpu_count()},
            "sample": f"numpy oracle of the full C1 step (Format Q pack of 3968 tokens x 8 heads + "
                      f"float32 attention of 32 heads over 4096 tokens); median of {n1} calls "
                      f"({t1 * 1e3:.0f} ms) on 1 thread, {nn} calls ({tn * 1e3:.0f} ms) on "
                      f"{os.cpu_count()} threads"}


def run_c5(args):
    """C5: full decode step, Qwen3-4B geometry (36 layers, 32 / 8 heads of 128,
    hidden 2560, FFN 9728, vocabulary 151936) with random-init bf16 weights,
    batch 4, 65536-token context in polar_cache (production knobs: chunk 16,
    dynamic candidate ratio, CDS 0.3 / 8 / 8, sink 64, local 256, top-100,
    update interval 512, full-attention threshold 2048), sampling at
    temperature 0.6 / top-p 0.95 / top-k 20, seed 42."""
    import statistics
    import torch
    from zoomkv_revision_amd import decode_step as ds
    ds.apply_production_env()
    geo = ds.Qwen3Geometry()
    batch, context, interval, threshold = 4, 65536, 512, 2048
    dev = torch.device("cuda:0")
    max_new = args.warmup + args.steps + interval + 64
    t0 = time.perf_counter()
    model = ds.RandomQwen3(geo, dev, seed=42)

    def run_mode(offload: bool, kv_format: str = "bf16"):
        """Timed steps, then untimed steps up to and through the first flush
        (every `interval` tokens): the flush step's extra time, amortized."""
        t_setup = time.perf_counter()
        cache = ds.build_cache(geo, batch, context, max_new, interval, threshold, dev, offload=offload,
                               kv_format=kv_format)
        ds.fill_cache(cache, geo, batch, context, 43, dev)
        torch.cuda.synchronize()
        setup = time.perf_counter() - t_setup
        print(f"[c5] offload={offload} kv_format={kv_format}: cache built and filled in {setup:.1f} s",
              file=sys.stderr, flush=True)
        gen = torch.Generator(device=dev)
        gen.manual_seed(42)
        state = {"tok": torch.randint(0, geo.vocab, (batch,), generator=gen, device=dev)}

        def step(i):
            logits = model.decode_step(state["tok"], cache)
            state["tok"] = ds.sample_next_token(logits, 0.6, 0.95, 20, generator=gen)

        ms = timed_loop(step, args.steps, args.warmup)
        print(f"[c5] offload={offload}: {ms:.3f} ms per step; stepping to the first flush", file=sys.stderr,
              flush=True)
        flushes_timed = cache._decode_step_counter // interval
        # step until the flush has run, timing each step (host clock, synchronised)
        times, flush_ms, i = [], None, args.warmup + args.steps
        while flush_ms is None and i < max_new - 1 and not args.no_flush:
            before = cache.cpu_valid_end[0]
            t1 = time.perf_counter()
            step(i)
            torch.cuda.synchronize()
            dt = (time.perf_counter() - t1) * 1e3
            if cache.cpu_valid_end[0] != before:
                flush_ms = dt
            else:
                times.append(dt)
            i += 1
        plain = statistics.median(times[-64:]) if times else ms
        extra = None if flush_ms is None else flush_ms - plain
        return cache, step, ms, setup, {
            "flushes_in_timed_region": flushes_timed,
            "flush_step_ms": flush_ms, "plain_step_ms": plain, "flush_extra_ms": extra,
            "flush_amortized_ms_per_step": None if extra is None else extra / interval,
            "per_token_latency_with_flush_ms": None if extra is None else ms + extra / interval,
        }

    qs = [torch.randn(batch, 1, geo.heads, geo.head_dim, device=dev).to(torch.bfloat16) for _ in range(geo.layers)]

    def attention_pass_ms(cache):
        """Device time of the attention path alone (36 x cache.compute)."""
        def attn_pass(i):
            for ldx in range(geo.layers):
                cache.compute(qs[ldx], ldx)
        return kernel_batch_ms(attn_pass, 8, host_us=15000.0)

    # the retrieval zone in device memory (the 288 GB part holds it)
    cache, step, ms, setup_dev, flush_dev = run_mode(False)
    setup_s = time.perf_counter() - t0
    flushes = flush_dev["flushes_in_timed_region"]
    # device time of one step and of its attention path alone, each queued
    # behind a spin kernel so host launch gaps are not counted
    step_ms = kernel_batch_ms(step, 8, host_us=20000.0)
    attn_ms = attention_pass_ms(cache)
    per_layer = [ds.attention_path_bytes(cache, ldx) for ldx in range(geo.layers)]
    attn_bytes = sum(p["total"] for p in per_layer)
    footprint = ds.cache_footprint(cache)
    weight_bytes = model.parameter_bytes()
    del cache, step
    torch.cuda.empty_cache()
    # the 4-bit K + V retrieval zone (kv_format="kivi4"): same selection,
    # token-list 4-bit attention
    kivi4 = None
    if not args.no_kivi4:
        cache_q, step_q, ms_q, setup_q, flush_q = run_mode(False, "kivi4")
        step_q_ms = kernel_batch_ms(step_q, 8, host_us=20000.0)
        attn_q_ms = attention_pass_ms(cache_q)
        per_layer_q = [ds.attention_path_bytes(cache_q, ldx) for ldx in range(geo.layers)]
        bytes_q = sum(p["total"] for p in per_layer_q)
        kivi4 = {"ms_per_step": ms_q, "tokens_per_s": batch / (ms_q * 1e-3), "setup_s": setup_q,
                 "device_ms_per_step": step_q_ms, **flush_q,
                 "attention_path": {"device_ms_per_step": attn_q_ms, "bytes_per_step": bytes_q,
                                    "GBps": bytes_q / (attn_q_ms * 1e-3) / 1e9,
                                    "bytes_per_layer": per_layer_q[0]},
                 "footprint_bytes": ds.cache_footprint(cache_q),
                 "per_token_floor_ms": (weight_bytes + bytes_q) / (HBM_PEAK_GBS * 1e9) * 1e3}
        kivi4["per_token_floor_frac"] = kivi4["per_token_floor_ms"] / ms_q
        del cache_q, step_q
        torch.cuda.empty_cache()
    # the reference runner's enable_offload=True: retrieval zone in pinned host memory
    offload = None
    if not args.no_offload:
        cache_h, step_h, ms_h, setup_h, flush_h = run_mode(True)
        offload = {"ms_per_step": ms_h, "tokens_per_s": batch / (ms_h * 1e-3), "setup_s": setup_h, **flush_h,
                   "host_bytes_pinned": sum(t.numel() * t.element_size()
                                            for t in cache_h.unified_keys_cpu + cache_h.unified_values_cpu)}
        del cache_h, step_h
        torch.cuda.empty_cache()
    return {
        "metric": "C5 full decode step (Qwen3-4B geometry, 36 layers): per-token latency, tokens/s",
        "value": batch / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 model; 4-bit K (Format R) stage-2 scoring + bf16 K/V attention",
        "data": "synthetic (random-init weights seed 42; cache prefilled with seeded N(0,1) K/V)",
        "config": {"workload": "C5: one decode token through 36 layers + sampling, polar_cache sparse path",
                   "batch": batch, "context": context, "layers": geo.layers, "hidden": geo.hidden,
                   "ffn": geo.ffn, "vocab": geo.vocab, "q_heads": geo.heads, "kv_heads": geo.kv_heads,
                   "head_dim": geo.head_dim, "update_interval": interval, "full_attention_threshold": threshold,
                   "sampling": {"temperature": 0.6, "top_p": 0.95, "top_k": 20, "seed": 42},
                   "attention_path": "polar_cache.compute: Quest stage 1 + KIVI 4-bit stage 2 (dense = sparse "
                                     "per-chunk top-k 8, so no density classification) + top-100 + "
                                     "gather-free bf16 attention",
                   "parallelism": "single GPU"},
        "per_token_latency_ms": ms,
        # weights + attention-path bytes at 8 TB/s, and the step's fraction of it
        "per_token_floor_ms": (weight_bytes + attn_bytes) / (HBM_PEAK_GBS * 1e9) * 1e3,
        "per_token_floor_frac": (weight_bytes + attn_bytes) / (HBM_PEAK_GBS * 1e9) * 1e3 / ms,
        "footprint_bytes": footprint,
        "kivi4_mode": kivi4,
        "flushes_in_timed_region": flushes,
        "flush": {k: v for k, v in flush_dev.items() if k != "flushes_in_timed_region"},
        "offload_mode": offload,
        "device_ms_per_step": step_ms,
        "attention_path": {"device_ms_per_step": attn_ms, "bytes_per_step": attn_bytes,
                           "GBps": attn_bytes / (attn_ms * 1e-3) / 1e9,
                           "bytes_per_layer": per_layer[0]},
        "weight_bytes_per_step": weight_bytes,
        "roofline": {"bound": "hbm", "achieved": attn_bytes / (attn_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": attn_bytes / (attn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "traffic": None, "kernel": "attention path (36 x polar_cache.compute)",
                     "kernel_ms": attn_ms, "algorithmic_bytes": attn_bytes},
        "setup_s": setup_s,
        "cpu_baseline": None,
    }


def run_h2d(args):
    """Host-to-device gather (the reference's UVA path, trans_h2d.py): the
    rows one decode layer gathers at C5's shape -- batch 4, 8 KV heads, 612
    rows per head (top-100 + 512 skipped) of a 65536-row pinned host cache."""
    import torch
    from zoomkv_revision_amd.gather import h2d_gather_kv
    bs, heads, src_len, topk = 4, 8, 65536, 612
    dev = torch.device("cuda:0")
    sk = torch.randn(bs, heads, src_len, 128).to(torch.bfloat16).pin_memory()
    sv = torch.randn(bs, heads, src_len, 128).to(torch.bfloat16).pin_memory()
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    idxs = [torch.randint(0, src_len, (bs, heads, topk), generator=g, device=dev) for _ in range(8)]
    dk = torch.empty(bs, heads, topk, 128, dtype=torch.bfloat16, device=dev)
    dv = torch.empty_like(dk)

    def step(i):
        h2d_gather_kv(sk, sv, idxs[i % len(idxs)], dk, dv)

    ms = timed_loop(step, args.steps, args.warmup)
    k_ms = kernel_batch_ms(step, args.steps)
    nbytes = bs * heads * topk * 2 * 256
    return {
        "metric": "host-to-device K/V row gather (pinned host cache): GB/s over the host link",
        "value": nbytes / (k_ms * 1e-3) / 1e9, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 rows", "data": "synthetic",
        "config": {"workload": "h2d_gather_kv: 612 rows of 256 B per (b, kv head), K and V",
                   "batch": bs, "kv_heads": heads, "src_len": src_len, "rows": topk,
                   "parallelism": "single GPU"},
        "kernel_ms": k_ms, "bytes_per_call": nbytes, "cpu_baseline": None,
    }


def run_c3(args):
    """C3: GQA-mean query + Quest bounds over fp16 page metadata (2048 pages of
    16 tokens, one launch) -> top-128 pages -> page-sparse 4-bit attention,
    batch 8, 32/8 heads, 32768 tokens; eight planted workloads rotate between
    steps (8 x 86 MB touched per step: Quest metadata 67.6 MB plus the selected
    pages, more than the 256 MB last-level cache)."""
    import numpy as np
    import torch
    from zoomkv_revision_amd import kivi, synthetic
    from zoomkv_revision_amd.quest import QuestTopkPlan, quest_chunk_topk_gqa
    bs, hq, kv, n_tok, n_sel = 8, 32, 8, 32768, 128
    dev = torch.device("cuda:0")
    ws = [synthetic.c3_workload(100 + i, bs, hq, kv, n_tok, n_sel, dev) for i in range(8)]
    n_pages = ws[0]["n_pages"]
    scores = torch.empty(bs, kv, n_pages, device=dev)
    raw_q = torch.empty(bs, kv, 128, dtype=torch.bfloat16, device=dev)
    sels = [torch.empty(bs, kv, n_sel, dtype=torch.int64, device=dev) for _ in range(2)]
    out = torch.empty(bs, hq, 128, dtype=torch.bfloat16, device=dev)
    sel_ok = []

    def select(i):
        # GQA mean + Quest bounds + top-128 pages: one launch
        w = ws[i % len(ws)]
        return quest_chunk_topk_gqa(w["q"], kv, w["page_min"], w["page_max"], scores, n_pages, None, raw_q, n_sel,
                                    sels[i % 2])

    # a decode loop runs the same buffers every step: the argument checks run
    # once per workload (QuestTopkPlan, SparseAttentionPlan), a step is two
    # C-ABI calls
    qplans = [QuestTopkPlan(w["q"], kv, w["page_min"], w["page_max"], scores, n_pages, None, raw_q, n_sel,
                            sels[j % 2]) for j, w in enumerate(ws)]
    splans = [kivi.SparseAttentionPlan(w["q"], w["cache"], sels[j % 2], out=out) for j, w in enumerate(ws)]

    def step(i):
        j = i % len(ws)
        qplans[j].run()
        splans[j].run()

    # the selection of every workload through the timed path's plans, checked
    # against its planted pages (outside the timed steps)
    for j in range(len(ws)):
        sel_ok.append(qplans[j].run().clone())
    ms = timed_loop(step, args.steps, args.warmup)
    step_ms = kernel_batch_ms(step, args.steps, host_us=60)
    k_ms = kernel_batch_ms(select, args.steps)
    sa_ms = kernel_batch_ms(lambda i: kivi.kivi4_sparse_attention(ws[i % len(ws)]["q"], ws[i % len(ws)]["cache"],
                                                                  ws[i % len(ws)]["planted"], out=out),
                            args.steps, host_us=30)
    exact = all(torch.equal(s, ws[j]["planted"]) for j, s in enumerate(sel_ok[:len(ws)]))
    nb = synthetic.c3_algorithmic_bytes(bs, hq, kv, n_pages, n_sel)
    achieved = nb["quest"] / (k_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        cpu = c3_cpu_baseline(ws[0], n_sel)
    return {
        "metric": "C3 Quest page select + sparse 4-bit attention: decode tokens/s",
        "value": bs / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16 metadata / u4->fp16 (fp32 accumulate)",
        "data": "synthetic (planted pages)",
        "config": {"workload": "C3: GQA mean + Quest (fp16 page min/max) + top-128 of 2048 pages (one "
                               "launch) -> page-sparse 4-bit attention", "batch": bs, "q_heads": hq,
                   "kv_heads": kv, "context": n_tok, "page_tokens": 16, "pages_selected": n_sel,
                   "parallelism": "single GPU"},
        "selection_equals_planted": exact,
        "end_to_end_GBps": nb["total"] / (ms * 1e-3) / 1e9,
        # the step's longest kernel: the fused GQA mean + Quest bounds + top-128
        # launch over the fp16 page metadata
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic("c3_quest_topk_traffic.json"),
                     "kernel": "quest_topk_kernel (GQA mean + Quest + top-128 pages)", "kernel_ms": k_ms,
                     "algorithmic_bytes": nb["quest"]},
        "algorithmic_bytes_per_step": nb,
        # device time of back-to-back steps (two launches each)
        "step_device_ms": step_ms,
        "step_GBps": nb["total"] / (step_ms * 1e-3) / 1e9,
        # the page-sparse attention: latency-bound (each wave's two paired
        # tiles land together after the page walk, then the wave and split
        # merges), so below its HBM line
        "sparse_attention": {"kernel_ms": sa_ms, "algorithmic_bytes": nb["sparse_attention"],
                             "GBps": nb["sparse_attention"] / (sa_ms * 1e-3) / 1e9},
        "cpu_baseline": cpu,
    }


def c3_cpu_baseline(w, n_sel, budget_s: float = 10.0):
    """The torch-CPU restatement of the C3 step (oracle/torch_cpu.py: Quest
    bounds over the fp16 page metadata, torch.topk, unpack + dequant of the
    selected pages, float32 SDPA with grouped heads) at the full C3 shape
    (batch 8, 32 / 8 heads, 2048 pages, top-128), timed with 1 thread and
    with every thread of the process's CPU share."""
    import numpy as np
    import torch
    from oracle import torch_cpu
    f16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
    c = w["cache"]
    prep = torch_cpu.prepare_c3(w["raw_q"].float().cpu().numpy(), f16(w["page_min"]), f16(w["page_max"]),
                                c.k_codes.cpu().numpy(), f16(c.k_meta), c.v_codes.cpu().numpy(), f16(c.v_meta))
    q = w["q"].float().cpu()
    sel, _ = torch_cpu.c3_step(q, prep, n_sel, 1 / math.sqrt(D))
    planted = torch.equal(sel, w["planted"].cpu())
    res = time_cpu_threads(lambda: torch_cpu.c3_step(q, prep, n_sel, 1 / math.sqrt(D)), budget_s)
    n_all = max(res)
    (t1, n1), (tn, nn) = res[1], res[n_all]
    bs = q.shape[0]
    return {"value": bs / t1, "unit": "tokens/s", "cores": 1, "kind": "port",
            "all_cores": {"value": bs / tn, "cores": n_all},
            "cpu_model": cpu_model(), "host_logical_cpus": os.cpu_count(),
            "sample": f"torch-CPU restatement (oracle/torch_cpu.py) of the whole C3 step at its full shape "
                      f"(batch {bs}, Quest over {prep['pmin'].shape[2]} pages, top-{n_sel}, sparse attention; selection equals "
                      f"the planted pages: {planted}); median of {n1} calls ({t1 * 1e3:.0f} ms) on 1 thread "
                      f"and {nn} calls ({tn * 1e3:.0f} ms) on {n_all} threads (the process's CPU share; "
                      f"host {os.cpu_count()} logical CPUs, {cpu_model()})"}


def run_c4(args):
    """C4: RaBitQ search, 131072 clustered unit keys (16-byte sign codes + fp16
    factors), 64 queries, top-256 by estimate, exact fp16 rerank; 80 key pools
    rotate between steps (each pass reads ~7 MB, below the 256 MB MALL)."""
    import torch
    from zoomkv_revision_amd import rabitq, synthetic
    n, nq, topk, n_pools = 131072, 64, 256, 80
    dev = torch.device("cuda:0")
    signs = rabitq.srht_signs(42, dev)
    pools = []
    for i in range(n_pools):
        keys = synthetic.c4_keys(1000 + i, n, 64, dev)
        codes, fac = rabitq.rabitq_encode(keys, signs)
        pools.append((keys, codes, fac))
    qs = synthetic.c4_keys(7, nq, 64, dev)
    ws = rabitq.search_workspace(1, nq, n, topk, dev)
    outs = (torch.empty(nq, topk, dtype=torch.int64, device=dev), torch.empty(nq, topk, dtype=torch.int64, device=dev),
            torch.empty(nq, topk, dtype=torch.float32, device=dev))

    # a serving loop searches the same buffers every step: the argument
    # checks run once per pool (rabitq.SearchPlan), each step is one C-ABI call
    plans = [rabitq.SearchPlan(qs, keys, codes, fac, signs, topk, workspace=ws, out=outs)
             for keys, codes, fac in pools]

    def step(i):
        plans[i % n_pools].run()

    ms = timed_loop(step, args.steps, args.warmup)
    k_ms = kernel_batch_ms(lambda i: rabitq.rabitq_search(qs, *pools[i % n_pools][:3], signs, topk, workspace=ws),
                           args.steps)
    algo = n * 20 + nq * topk * 256 + nq * 128 * 2 + nq * topk * 20
    achieved = algo / (k_ms * 1e-3) / 1e9
    cpu = None if args.no_cpu else c4_cpu_baseline(pools[0], qs, signs, topk)
    return {
        "metric": "C4 RaBitQ 1-bit search: queries/s (top-256 of 131072 + exact rerank)",
        "value": nq / (ms * 1e-3), "unit": "queries/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u1 codes (popcount) + fp16 rerank (fp32 accumulate)",
        "data": "synthetic (seeded unit-norm clusters)",
        "config": {"workload": "C4: encode queries -> estimate + exact top-256 -> fp16 rerank",
                   "keys": n, "queries": nq, "topk": topk, "clusters": 64, "pools_rotated": n_pools,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic("c4_rabitq_search_traffic.json"),
                     "kernel": "rabitq_search (prep + filter + select)", "kernel_ms": k_ms,
                     "algorithmic_bytes": algo},
        "cpu_baseline": cpu,
    }


def c4_cpu_baseline(pool, qs, signs, topk, budget_s: float = 10.0):
    """The torch-CPU restatement of the C4 search (oracle/torch_cpu.py: query
    rotation and codes, XOR + 64-bit bit count over the 131072 key codes for
    all 64 queries, torch.topk, exact fp32 rerank) at the full C4 shape,
    timed with 1 thread and with every thread of the process's CPU share."""
    import numpy as np
    import torch
    from oracle import torch_cpu
    keys, codes, fac = pool
    f16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
    prep = torch_cpu.prepare_c4(f16(keys), codes.cpu().numpy(), f16(fac), signs.cpu().numpy())
    q = qs.float().cpu()
    res = time_cpu_threads(lambda: torch_cpu.c4_search(q, prep, topk), budget_s)
    n_all = max(res)
    (t1, n1), (tn, nn) = res[1], res[n_all]
    nq = q.shape[0]
    return {"value": nq / t1, "unit": "queries/s", "cores": 1, "kind": "port",
            "all_cores": {"value": nq / tn, "cores": n_all},
            "cpu_model": cpu_model(), "host_logical_cpus": os.cpu_count(),
            "sample": f"torch-CPU restatement (oracle/torch_cpu.py) of the whole C4 search at its full shape "
                      f"({nq} queries x {keys.shape[0]} keys, top-{topk} + exact rerank); median of {n1} calls "
                      f"({t1 * 1e3:.0f} ms) on 1 thread and {nn} calls ({tn * 1e3:.0f} ms) on {n_all} threads "
                      f"(the process's CPU share; host {os.cpu_count()} logical CPUs, {cpu_model()})"}


def run_r4(args):
    """R4: ParisKV 4-bit RaBitQ codes (1-bit sign + 3-bit magnitude) at the
    decode shape the reference's rerank module documents
    (Z/cache_hub/rerank/rerank.py:1-20: one layer, kv_len ~128K, ~13K
    candidates (10%), final_topk 100).  Per step: the 8 KV heads' queries to
    SRHT blocks, the 4-bit approximate scores of the candidates, and their
    top-100 key indices.  4 caches rotate between steps (96 MB of codes and
    weights each in the reference's [16, seq] layout: 384 MB > the MALL)."""
    import torch
    from zoomkv_revision_amd import rabitq4
    bs, kv, L, C, k, n_caches = 1, 8, 131072, 13108, 100, 4
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(42)
    signs = (torch.randint(0, 2, (128,), device=dev, generator=gen) * 2 - 1).to(torch.bfloat16)
    thr, ctr = rabitq4.magnitude_levels(device=dev)
    caches = []
    for i in range(n_caches):
        keys = torch.randn(bs, kv, L, 128, device=dev, generator=gen).to(torch.bfloat16)
        code, w, packed = rabitq4.batch_encode(keys, signs, thr, ctr)
        cand = torch.stack([torch.randperm(L, device=dev, generator=gen)[:C] for _ in range(kv)]).view(bs, kv, C)
        caches.append((packed, w, cand))
    keys = torch.randn(bs, kv, L, 128, device=dev, generator=gen).to(torch.bfloat16)
    q = torch.randn(bs, kv, 128, device=dev, generator=gen).to(torch.bfloat16)
    f32 = torch.empty(bs, kv, C, dtype=torch.float32, device=dev)

    def step(i):
        packed, w, cand = caches[i % n_caches]
        qb, qn = rabitq4.encode_query_blocks(q, signs)
        return rabitq4.rabitq_rerank_topk(cand, packed, w, qb, qn, ctr, k)

    ms = timed_loop(step, args.steps, args.warmup)
    qb, qn = rabitq4.encode_query_blocks(q, signs)
    k_ms = kernel_batch_ms(lambda i: rabitq4._rerank(caches[i % n_caches][2], caches[i % n_caches][0],
                                                     caches[i % n_caches][1], qb, qn, ctr, 16, 8, scores_f32=f32),
                           args.steps)
    code_o = torch.empty(bs, kv, 16, L, dtype=torch.uint8, device=dev)
    w_o = torch.empty(bs, kv, 16, L, dtype=torch.bfloat16, device=dev)
    p_o = torch.empty(bs, kv, 16, L, 4, dtype=torch.uint8, device=dev)
    enc_ms = kernel_batch_ms(lambda i: rabitq4.encode_into(keys, signs, thr, ctr, code_o, w_o, p_o, 0), 5)
    # Algorithmic bytes of one rerank call: every 64-byte sector of codes
    # (16 tokens x 4 B per block) and of weights (32 tokens x 2 B per block)
    # that holds a candidate -- the least any reader of the [16, seq] layout
    # moves -- plus the candidate indices in and the fp32 scores out.  The
    # figure is averaged over the rotated caches' candidate sets.
    sectors = 0
    for _, _, cand in caches:
        for h in range(kv):
            t = cand[0, h]
            sectors += 16 * (torch.unique(t // 16).numel() + torch.unique(t // 32).numel())
    algo = 64 * sectors // n_caches + C * kv * (8 + 4) + kv * (256 + 2)
    achieved = algo / (k_ms * 1e-3) / 1e9
    enc_bytes = bs * kv * L * (256 + 16 * 7)      # bf16 key in; sign byte, code word, weight out per block
    cpu = None if args.no_cpu else r4_cpu_baseline(caches[0], q, signs, k)
    return {
        "metric": "R4 ParisKV 4-bit RaBitQ rerank + top-100 per decode step: candidates/s",
        "value": C * kv / (ms * 1e-3), "unit": "candidates/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4 codes (sign + 3-bit magnitude) -> bf16 (sequential bf16 sums)",
        "data": "synthetic (seeded N(0,1) keys and queries, random candidate sets)",
        "config": {"workload": "R4: query SRHT blocks -> 4-bit scores of the candidates -> top-100 key indices",
                   "batch": bs, "kv_heads": kv, "keys": L, "candidates": C, "topk": k,
                   "caches_rotated": n_caches, "layout": "reference [16, seq] codes and weights",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic("r4_rabitq4_rerank_traffic.json"),
                     "kernel": "rabitq4 rerank call (mark + stream + collect kernels)", "kernel_ms": k_ms,
                     "algorithmic_bytes": algo},
        "key_encode": {"keys_per_s": bs * kv * L / (enc_ms * 1e-3), "kernel_ms": enc_ms,
                       "GBps": enc_bytes / (enc_ms * 1e-3) / 1e9, "keys": bs * kv * L},
        "cpu_baseline": cpu,
    }


def r4_cpu_baseline(cache, q, signs, k, budget_s: float = 10.0):
    """The numpy oracle (oracle/rabitq4.py) of one step for 1 of the 8 heads."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits
    from oracle import rabitq4 as r4
    from oracle.numerics import bf16_to_f32
    packed, w, cand = cache
    tb = lambda t: bf16_to_f32(t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16))
    p_np, w_np, c_np = packed[0, 0].cpu().numpy(), tb(w[0, 0]), cand[0, 0].cpu().numpy()
    q_np, s_np = tb(q[0, 0]), tb(signs)
    times = []
    with threadpool_limits(limits=1):
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(times) < 2:
            t0 = time.perf_counter()
            qb, qn = r4.encode_query(q_np, s_np)
            sc = r4.rerank_scores(c_np, p_np, w_np, qb, qn)
            r4.topk_gather(sc, c_np, k)
            times.append(time.perf_counter() - t0)
            if len(times) >= 20:
                break
    t = statistics.median(times)
    return {"value": c_np.shape[0] / t, "unit": "candidates/s", "cores": 1, "kind": "port",
            "sample": f"numpy oracle step (query blocks, 4-bit scores of {c_np.shape[0]} candidates, top-{k}) "
                      f"for 1 of the 8 KV heads; median of {len(times)} calls ({t * 1e3:.0f} ms each); "
                      f"host {os.cpu_count()} logical CPUs, 1 used"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default 150 for c2: ~16 ms of streaming, past the power "
                         "manager's transient, so the timed steps see the settled clock; 10 otherwise)")
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--config", choices=["c1", "c2", "c3", "c4", "c5", "r4", "h2d"], default="c2",
                    help="c2 (default, the headline line), c1, c3, c4, c5, r4 (ParisKV 4-bit RaBitQ) or h2d")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-offload", action="store_true",
                    help="c5: skip the run with the retrieval zone in pinned host memory")
    ap.add_argument("--no-kivi4", action="store_true",
                    help="C5: skip the 4-bit K + V retrieval-zone mode")
    ap.add_argument("--no-flush", action="store_true",
                    help="c5: skip stepping to the first flush (its timing)")
    ap.add_argument("--hbm-reference", action="store_true",
                    help="c2: only compare the attention's stream rate with torch's device copy and "
                         "torch.sum over the same byte volume (medians of 6 interleaved rounds) and exit")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 5 device copies of 1 GiB (scale reference for rocprof "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.warmup is None:
        args.warmup = 150 if args.config == "c2" else 10
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build runs on a "
              "single MI355X and the path shards per (batch, kv head) with no exchange", file=sys.stderr)
        sys.exit(2)

    import torch
    from zoomkv_revision_amd import kivi
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.config != "c2":
        run = {"c1": run_c1, "c3": run_c3, "c4": run_c4, "c5": run_c5, "r4": run_r4, "h2d": run_h2d}[args.config]
        print(json.dumps(run(args)))
        return
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)      # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4}))
        return
    caches = [make_cache(1234 + i, dev) for i in range(2)]
    from zoomkv_revision_amd import synthetic
    if args.hbm_reference:
        print(json.dumps(hbm_reference(caches, synthetic.c2_query(B, HQ, dev))))
        return
    q = synthetic.c2_query(B, HQ, dev)
    out = torch.empty(B, HQ, D, dtype=torch.bfloat16, device=dev)
    ws = kivi.attention_workspace(B, HQ, HKV, NG, R, args.splits, device=dev)
    torch.cuda.synchronize()

    def step(i):
        # one launch: the context splits, merged by the workgroup that
        # completes each (sequence, KV head)
        kivi.kivi4_decode_attention(q, caches[i % 2], NG, R, out=out, n_splits=args.splits, workspace=ws)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # the dominant kernel's mean launch time: HIP events on the launch stream
    # (torch's current stream, which the C-ABI call receives) bracketing the
    # timed steps themselves (the host enqueues ~10 us per step ahead of the
    # ~108 us launches, so the device runs them back to back)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for i in range(args.steps):
        step(i)
    ev1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    k_ms = ev0.elapsed_time(ev1) / args.steps
    # sustained load: 240 back-to-back launches, the settled median of the last 100
    sus = sustained_ms(step)
    _, used = kivi.kivi4_attention_partial(q, caches[0], NG, R, n_splits=args.splits, workspace=ws)  # the plan
    achieved = ALGO_BYTES / (k_ms * 1e-3) / 1e9
    sus_achieved = ALGO_BYTES / (sus["sustained_ms"] * 1e-3) / 1e9

    cpu = None if args.no_cpu else cpu_baseline(caches[0], q)
    line = {
        "metric": METRIC,
        "value": B / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u4->fp16 (fp32 accumulate)", "data": "synthetic",
        "config": {"workload": "C2: fused 4-bit KV decode attention (Format Q cache + bf16 residual)",
                   "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": T,
                   "quantized_tokens": NG * 32, "residual_tokens": R, "k_group_tokens": 32,
                   "v_group_channels": 32, "splits": used, "parallelism": "single GPU"},
        "kv_tokens_per_s": B * T / (ms_step * 1e-3),
        "end_to_end_GBps": ALGO_BYTES / (ms_step * 1e-3) / 1e9,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": read_traffic(),
                     "kernel": "kivi4_attn_kernel", "kernel_ms": k_ms,
                     "algorithmic_bytes": ALGO_BYTES},
        # the same kernel under sustained load (the clock settles lower after
        # ~2 ms of full-bandwidth streaming): per-launch medians of 240
        # back-to-back launches
        "sustained": {"launches": sus["launches"], "burst_kernel_ms": sus["burst_ms"],
                      "settled_kernel_ms": sus["sustained_ms"], "settled_tokens_per_s": B / (sus["sustained_ms"] * 1e-3),
                      "settled_GBps": sus_achieved, "settled_frac": sus_achieved / HBM_PEAK_GBS,
                      "max_kernel_ms": sus["max_ms"]},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
