"""CDS density scores, dense mask and the GQA-mean query over the gfx950 C ABI.

Names and arguments follow Z/cache_hub/rerank/rerank.py:587-633 (the ``kernel``
argument is accepted and ignored: the native library is loaded once).
"""
from __future__ import annotations

import torch

from ._lib import check, lib, ptr, require_gpu, stream_of


def partial_chunk_density_scores_cuda(chunk_ids: torch.Tensor, chunk_centroids: torch.Tensor,
                                      raw_q: torch.Tensor, out_scores: torch.Tensor,
                                      kernel=None) -> None:
    """out[b, h, j] = centroid[b, h, chunk_ids[b, h, j]] . raw_q[b, h]; -1e30 for bad ids."""
    require_gpu(chunk_ids, chunk_centroids, raw_q, out_scores)
    if chunk_centroids.dtype != torch.bfloat16:
        chunk_centroids = chunk_centroids.to(torch.bfloat16)
    if raw_q.dtype != torch.bfloat16:
        raw_q = raw_q.to(torch.bfloat16)
    if out_scores.dtype != torch.float32:
        raise TypeError(f"out_scores must be float32, got {out_scores.dtype}")
    if chunk_ids.dtype != torch.int64:
        raise RuntimeError("chunk_ids must be int64")
    bs, kv, nk = chunk_ids.shape
    n_chunks = chunk_centroids.shape[2]
    for t in (chunk_ids, chunk_centroids, raw_q, out_scores):
        if t.stride(-1) != 1:
            raise RuntimeError("last dims must be contiguous")
    if chunk_centroids.shape[3] != 128 or raw_q.shape[2] != 128:
        raise RuntimeError("head_dim must be 128")
    check(lib().zkv_chunk_density_scores(
        ptr(chunk_ids), chunk_ids.stride(0), chunk_ids.stride(1),
        ptr(chunk_centroids), chunk_centroids.stride(0), chunk_centroids.stride(1),
        chunk_centroids.stride(2), ptr(raw_q), raw_q.stride(0), raw_q.stride(1),
        ptr(out_scores), out_scores.stride(0), out_scores.stride(1), bs, kv, nk, n_chunks,
        stream_of(raw_q)))


def dense_mask_from_topk_cuda(positions: torch.Tensor, mask: torch.Tensor, kernel=None) -> None:
    """mask.fill_(False); mask.scatter_(2, positions, True) in one kernel."""
    require_gpu(positions, mask)
    positions = positions.contiguous()
    if positions.dtype != torch.int64 or mask.dtype != torch.bool or not mask.is_contiguous():
        raise RuntimeError("positions must be int64 and mask a contiguous bool tensor")
    bs, kv, nk = mask.shape
    check(lib().zkv_dense_mask_from_topk(ptr(positions), ptr(mask), bs * kv, positions.shape[-1], nk,
                                         stream_of(mask)))


def topk_dense_mask(scores: torch.Tensor, k: int, mask: torch.Tensor, out: torch.Tensor | None = None):
    """dense_mask_from_topk_cuda(float_topk_3d(scores, k), mask) in one launch:
    scores [bs, kv, L] fp32, mask [bs, kv, L] bool; returns the top-k indices."""
    require_gpu(scores, mask)
    bs, kv, L = scores.shape
    assert k <= L, "k must not exceed the row length"
    if scores.dtype != torch.float32 or scores.stride(-1) != 1 or scores.stride(0) != kv * scores.stride(1):
        scores = scores.float().contiguous()
    if mask.dtype != torch.bool or not mask.is_contiguous() or tuple(mask.shape) != (bs, kv, L):
        raise RuntimeError("mask must be a contiguous bool tensor [bs, kv, L]")
    if out is None:
        out = torch.empty(bs, kv, k, dtype=torch.int64, device=scores.device)
    check(lib().zkv_topk_dense_mask(ptr(scores), scores.stride(1), bs * kv, L, k, ptr(out), out.stride(1),
                                    ptr(mask), L, stream_of(scores)))
    return out


def gqa_mean_query(q: torch.Tensor, kv_heads: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """raw_q = q.view(bs, kv, g, 128).mean(2) in bf16 (S:1621-1626); q [bs, hq, 128] or [bs, 1, hq, 128]."""
    require_gpu(q)
    q3 = q[:, 0] if q.dim() == 4 else q
    if q3.dtype != torch.bfloat16 or q3.stride(-1) != 1 or q3.shape[-1] != 128:
        raise RuntimeError("q must be bf16 with a contiguous last dim of 128")
    bs, hq, _ = q3.shape
    if out is None:
        out = torch.empty(bs, kv_heads, 128, dtype=torch.bfloat16, device=q.device)
    check(lib().zkv_gqa_mean_query(ptr(q3), q3.stride(0), q3.stride(1), bs, hq, kv_heads, ptr(out),
                                   stream_of(q)))
    return out
