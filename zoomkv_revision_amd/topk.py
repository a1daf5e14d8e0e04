"""Exact top-k and the fused top-k + gather + skipped-tail concat (gfx950).

``float_topk`` / ``float_topk_3d`` mirror Z/cache_hub/topk/float_topk_ops.py:63-106
and ``float_topk_gather_concat_3d`` mirrors
Z/cache_hub/topk/float_topk_gather_concat_ops.py:77-125.  The reference's radix
select returns the top-k set in arbitrary order (and may drop candidates when
more than 8192 share a radix bucket, float_topk.cu:95); these return the exact
top-k set, ties broken by lowest index, in increasing index order.
"""
from __future__ import annotations

import math

import torch

from ._lib import check, lib, ptr, require_gpu, stream_of


def _rows(t: torch.Tensor) -> torch.Tensor:
    """A view whose rows (all but the last dim) are equally strided, last dim contiguous."""
    if t.stride(-1) != 1:
        return t.contiguous()
    if t.dim() == 3 and t.stride(0) != t.shape[1] * t.stride(1):
        return t.contiguous()
    return t


def _topk(scores: torch.Tensor, k: int, out: torch.Tensor, lut=None, skipped=None, sentinel=-1):
    L = scores.shape[-1]
    rows = math.prod(scores.shape[:-1])
    sk = 0 if skipped is None else skipped.shape[-1]
    check(lib().zkv_topk(
        ptr(scores), scores.stride(-2), rows, L, int(k), ptr(out), out.stride(-2),
        ptr(lut), 0 if lut is None else lut.stride(-2),
        ptr(skipped) if sk else None, 0 if not sk else skipped.stride(-2), sk, int(sentinel),
        stream_of(scores)))
    return out


def float_topk(scores: torch.Tensor, k: int) -> torch.Tensor:
    """[B, L] float -> [B, k] int64 indices of the k largest (sentinel -1 if L <= k)."""
    require_gpu(scores)
    assert scores.dim() == 2, "scores must be 2D [B, L]"
    assert 0 < k <= scores.size(1), f"k={k} out of range"
    s = _rows(scores if scores.dtype == torch.float32 else scores.float())
    out = torch.empty(s.shape[0], k, dtype=torch.int64, device=s.device)
    return _topk(s, k, out)


def float_topk_3d(scores: torch.Tensor, k: int) -> torch.Tensor:
    """[bs, kv, L] float -> [bs, kv, k] int64."""
    require_gpu(scores)
    assert scores.dim() == 3, "scores must be 3D [bs, kv_heads, n_chunks]"
    assert 0 < k <= scores.size(2), f"k={k} cannot exceed n_chunks={scores.size(2)}"
    s = _rows(scores if scores.dtype == torch.float32 else scores.float())
    bs, kv, _ = s.shape
    out = torch.empty(bs, kv, k, dtype=torch.int64, device=s.device)
    return _topk(s, k, out)


def float_topk_gather_concat_3d(scores: torch.Tensor, lut: torch.Tensor, skipped: torch.Tensor,
                                out: torch.Tensor, k: int) -> torch.Tensor:
    """out[..., :k] = lut[topk(scores, k)], out[..., k:k+sk] = skipped; 0 sentinel."""
    require_gpu(scores, lut, skipped, out)
    assert scores.dim() == 3 and lut.dim() == 3 and skipped.dim() == 3 and out.dim() == 3
    assert scores.dtype == torch.float32, f"scores must be fp32; got {scores.dtype}"
    assert lut.dtype == torch.int64 and skipped.dtype == torch.int64 and out.dtype == torch.int64
    assert scores.shape == lut.shape, f"scores/lut shape mismatch: {scores.shape} vs {lut.shape}"
    assert skipped.shape[:2] == scores.shape[:2] and out.shape[:2] == scores.shape[:2]
    sk = skipped.shape[2]
    assert 0 < k <= scores.shape[2], f"k={k} out of range [1, {scores.shape[2]}]"
    assert out.shape[2] >= k + sk, f"out last dim={out.shape[2]} must be >= k+sk={k + sk}"
    assert out.is_contiguous(), "out must be contiguous"
    s, l = _rows(scores), _rows(lut)
    skp = _rows(skipped) if sk else skipped
    return _topk(s, k, out, lut=l, skipped=skp if sk else None, sentinel=0)
