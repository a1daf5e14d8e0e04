"""Seeded synthetic workloads of the benchmark configurations (no datasets or
checkpoints are available offline; shapes follow the reference's headline
configurations).

* C1: one layer, batch 1, 32 / 8 heads, 4096 tokens of N(0, 1) bf16 K / V with
  4 key channels x10 (the same channels for every head); the first 3968
  tokens (124 groups of 32) go to the 4-bit cache, the last 128 stay bf16.

* C2: Format Q cache of Gaussian bf16 K/V with 1% outlier K channels x10 plus
  a bf16 residual window (fused 4-bit decode attention).
* C3: paged 4-bit cache with per-page fp16 Quest min/max and planted pages:
  per (b, kv) ``n_plant`` random pages hold keys ``alpha * q_hat + 0.1 N(0, 1)``
  (q_hat the unit GQA-mean query), alpha large enough that every planted
  page's Quest bound clears every other page's, so the right selection is
  known.
* C4: unit-norm keys around seeded Gaussian cluster centres (RaBitQ search).
"""
from __future__ import annotations

import math

import torch

from . import kivi
from .quest import page_minmax_f16, quest_chunk_score
from .rerank import gqa_mean_query

HEAD_DIM = 128


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def c1_workload(seed: int = 42) -> dict:
    """C1 inputs on the CPU (torch.Generator seeded on the CPU, as the
    measurement definition asks): q [1, 32, 128], k / v [1, 8, 4096, 128]
    bf16, the outlier channels, and the quantized / residual split."""
    g = torch.Generator()
    g.manual_seed(seed)
    q = torch.randn(1, 32, HEAD_DIM, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 8, 4096, HEAD_DIM, generator=g)
    v = torch.randn(1, 8, 4096, HEAD_DIM, generator=g)
    ch = torch.randperm(HEAD_DIM, generator=g)[:4]
    k[..., ch] *= 10.0
    return {"q": q, "k": k.to(torch.bfloat16), "v": v.to(torch.bfloat16), "outlier_channels": ch,
            "n_quant": 3968, "n_groups": 124, "res_len": 128}


def c2_cache(seed: int, bs: int, kv: int, n_groups: int, res_len: int, device,
             outlier_frac: float = 0.01, keep_rows=()):
    """Format Q cache of n_groups * 32 Gaussian tokens (outlier K channels x10)
    plus res_len bf16 residual tokens, packed on the GPU one sequence at a time.

    With ``keep_rows`` (batch indices) it returns (cache, kept), kept[b] = the
    bf16 K and V of sequence b as host float32 arrays [1, kv, n_groups * 32,
    128], for checking the pack and the attention against a CPU model."""
    g = _gen(seed, device)
    cache = kivi.Kivi4Cache.allocate(bs, kv, n_groups, max(res_len, 1), device=device)
    n = n_groups * 32
    n_out = max(1, round(outlier_frac * HEAD_DIM))
    kept = {}
    for b in range(bs):
        k = torch.randn(kv, n, HEAD_DIM, generator=g, device=device)
        v = torch.randn(kv, n, HEAD_DIM, generator=g, device=device)
        for h in range(kv):
            ch = torch.randperm(HEAD_DIM, generator=g, device=device)[:n_out]
            k[h, :, ch] *= 10.0
        kb, vb = k.to(torch.bfloat16)[None], v.to(torch.bfloat16)[None]
        kivi.kivi4_pack(kb, vb, cache.rows(b, b + 1), 0)
        if b in keep_rows:
            kept[b] = (kb.float().cpu().numpy(), vb.float().cpu().numpy())
        del k, v, kb, vb
    if res_len:
        cache.k_res[:, :, :res_len].copy_(
            torch.randn(bs, kv, res_len, HEAD_DIM, generator=g, device=device).to(torch.bfloat16))
        cache.v_res[:, :, :res_len].copy_(
            torch.randn(bs, kv, res_len, HEAD_DIM, generator=g, device=device).to(torch.bfloat16))
    cache.n_groups, cache.res_len = n_groups, res_len
    return (cache, kept) if keep_rows else cache


def c2_query(bs: int, hq: int, device, seed: int = 42) -> torch.Tensor:
    """The C2 benchmark's query rows: bf16 [bs, hq, 128], N(0, 1), seeded on the device."""
    g = _gen(seed, device)
    return torch.randn(bs, hq, HEAD_DIM, generator=g, device=device).to(torch.bfloat16)


def c3_workload(seed: int, bs: int, hq: int, kv: int, n_tok: int, n_plant: int, device,
                page: int = 16, keep_keys: bool = False) -> dict:
    """Paged cache with planted pages.  Returns q bf16 [bs, hq, 128], raw_q
    (GQA mean), cache (Format Q, no residual), page_min / page_max fp16
    [bs, kv, n_pages, 128], planted int64 [bs, kv, n_plant] (sorted) and,
    with keep_keys, the bf16 keys / values."""
    assert n_tok % 32 == 0 and page == 16
    g = _gen(seed, device)
    n_pages = n_tok // page
    q = torch.randn(bs, hq, HEAD_DIM, generator=g, device=device).to(torch.bfloat16)
    raw_q = gqa_mean_query(q, kv)
    k = torch.randn(bs, kv, n_tok, HEAD_DIM, generator=g, device=device).to(torch.bfloat16)
    v = torch.randn(bs, kv, n_tok, HEAD_DIM, generator=g, device=device).to(torch.bfloat16)
    planted = torch.stack([torch.stack([torch.randperm(n_pages, generator=g, device=device)[:n_plant]
                                        for _ in range(kv)]) for _ in range(bs)])
    planted, _ = planted.sort(dim=-1)
    # alpha: 3x the largest unplanted Quest bound over ||raw_q||
    pmin, pmax = page_minmax_f16(k, page)
    scores = torch.empty(bs, kv, n_pages, device=device)
    quest_chunk_score(raw_q, pmin, pmax, scores, n_pages)
    qf = raw_q.float()
    qn = qf.norm(dim=-1, keepdim=True)
    alpha = 3.0 * scores.amax(dim=-1, keepdim=True).clamp_min(1.0) / qn           # [bs, kv, 1]
    tok = (planted[..., None] * page + torch.arange(page, device=device)).reshape(bs, kv, -1)
    noise = 0.1 * torch.randn(bs, kv, tok.shape[-1], HEAD_DIM, generator=g, device=device)
    pk = (alpha[..., None] * (qf / qn)[:, :, None, :] + noise).to(torch.bfloat16)
    k.scatter_(2, tok[..., None].expand(-1, -1, -1, HEAD_DIM), pk)
    pmin, pmax = page_minmax_f16(k, page)
    cache = kivi.Kivi4Cache.allocate(bs, kv, n_tok // 32, 1, device=device)
    kivi.kivi4_pack(k, v, cache, 0)
    cache.n_groups, cache.res_len = n_tok // 32, 0
    out = {"q": q, "raw_q": raw_q, "cache": cache, "page_min": pmin, "page_max": pmax,
           "planted": planted, "n_pages": n_pages}
    if keep_keys:
        out["k"], out["v"] = k, v
    return out


def c4_keys(seed: int, n: int, n_clusters: int, device, sigma: float = 0.1) -> torch.Tensor:
    """n unit-norm fp16 keys around n_clusters seeded Gaussian centres."""
    g = _gen(seed, device)
    centres = torch.randn(n_clusters, HEAD_DIM, generator=g, device=device)
    centres = centres / centres.norm(dim=1, keepdim=True)
    lab = torch.randint(0, n_clusters, (n,), generator=g, device=device)
    x = centres[lab] + sigma * torch.randn(n, HEAD_DIM, generator=g, device=device)
    return (x / x.norm(dim=1, keepdim=True)).to(torch.float16)


def c3_algorithmic_bytes(bs: int, hq: int, kv: int, n_pages: int, n_sel: int) -> dict:
    """Bytes of the C3 step's kernels by algorithm: the Quest metadata scan
    (with the GQA-mean query formed from the query heads and stored in the
    same launch), and the sparse attention's selected pages at 160 B per
    token (codes + metadata)."""
    quest = bs * kv * (n_pages * 2 * HEAD_DIM * 2 + n_pages * 4 + HEAD_DIM * 2) + bs * hq * HEAD_DIM * 2
    attn = bs * kv * n_sel * 16 * 160 + bs * hq * HEAD_DIM * 2 * 2
    return {"quest": quest, "sparse_attention": attn, "total": quest + attn}


def sm_scale() -> float:
    return 1.0 / math.sqrt(HEAD_DIM)
