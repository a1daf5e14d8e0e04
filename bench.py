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
kernel (HIP events on the launch stream over the timed region) and the CPU
baseline (the numpy oracle, one host thread, on a bounded sample).
"""
from __future__ import annotations

import argparse
import json
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
    import torch
    from zoomkv_revision_amd import kivi
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    cache = kivi.Kivi4Cache.allocate(B, HKV, NG, R, device=device)
    n = NG * 32
    n_out = max(1, round(0.01 * D))
    for b in range(B):
        k = torch.randn(HKV, n, D, generator=g, device=device, dtype=torch.float32)
        v = torch.randn(HKV, n, D, generator=g, device=device, dtype=torch.float32)
        for h in range(HKV):
            ch = torch.randperm(D, generator=g, device=device)[:n_out]
            k[h, :, ch] *= 10.0
        view = kivi.Kivi4Cache(cache.k_codes[b:b + 1], cache.k_meta[b:b + 1], cache.v_codes[b:b + 1],
                               cache.v_meta[b:b + 1], cache.k_res[b:b + 1], cache.v_res[b:b + 1])
        kivi.kivi4_pack(k.to(torch.bfloat16)[None], v.to(torch.bfloat16)[None], view, 0)
        del k, v
    cache.k_res.copy_(torch.randn(B, HKV, R, D, generator=g, device=device).to(torch.bfloat16))
    cache.v_res.copy_(torch.randn(B, HKV, R, D, generator=g, device=device).to(torch.bfloat16))
    cache.n_groups, cache.res_len = NG, R
    return cache


def cpu_baseline(cache, q, budget_s: float = 12.0):
    """Time the numpy oracle (dequant + softmax attention, float32, 1 thread) on
    sequence 0 of the batch: 1 of 16 sequences per call."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import kivi as okivi
    c0 = okivi.Kivi4Cache(cache.k_codes[:1].cpu().numpy(),
                          cache.k_meta[:1].cpu().view(__import__("torch").int16).numpy().view(np.uint16),
                          cache.v_codes[:1].cpu().numpy(),
                          cache.v_meta[:1].cpu().view(__import__("torch").int16).numpy().view(np.uint16))
    kr = cache.k_res[:1].float().cpu().numpy()
    vr = cache.v_res[:1].float().cpu().numpy()
    q0 = q[:1].float().cpu().numpy()
    times = []
    with threadpool_limits(limits=1):
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(times) < 2:
            t0 = time.perf_counter()
            okivi.kivi4_decode_attention(q0, c0, NG, kr, vr, R, 1 / np.sqrt(D), dtype=np.float32)
            times.append(time.perf_counter() - t0)
            if len(times) >= 20:
                break
    t = statistics.median(times)
    return {"value": 1.0 / t, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"numpy oracle (Format Q dequant + float32 softmax attention) on 1 of {B} "
                      f"sequences ({HKV} KV heads x {T} tokens) per call; median of {len(times)} "
                      f"calls ({t * 1e3:.0f} ms each); host {os.cpu_count()} logical CPUs, 1 used"}


def read_traffic():
    path = os.path.join(ROOT, "profiles", "kivi4_attn_c2_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--splits", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 5 device copies of 1 GiB (scale reference for rocprof "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build runs on a "
              "single MI355X and the path shards per (batch, kv head) with no exchange", file=sys.stderr)
        sys.exit(2)

    import torch
    from zoomkv_revision_amd import kivi
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)      # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4}))
        return
    caches = [make_cache(1234 + i, dev) for i in range(2)]
    gq = torch.Generator(device=dev)
    gq.manual_seed(42)
    q = torch.randn(B, HQ, D, generator=gq, device=dev).to(torch.bfloat16)
    out = torch.empty(B, HQ, D, dtype=torch.bfloat16, device=dev)
    ws = kivi.attention_workspace(B, HQ, HKV, NG, R, args.splits, device=dev)
    torch.cuda.synchronize()

    def step(i, ev=None):
        # the two kernels of kivi4_decode_attention: split attention, then the
        # LSE merge of the splits (events bracket the main kernel alone)
        if ev is not None:
            ev[0].record()
        _, used = kivi.kivi4_attention_partial(q, caches[i % 2], NG, R, n_splits=args.splits,
                                               workspace=ws)
        if ev is not None:
            ev[1].record()
        if used > 1:
            kivi.attention_merge(ws, B, HQ, HKV, used, out)
        return used

    for i in range(args.warmup):
        step(i)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        used = step(i, events[i])
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    k_ms = statistics.mean(a.elapsed_time(b) for a, b in events)
    achieved = ALGO_BYTES / (k_ms * 1e-3) / 1e9

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
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
