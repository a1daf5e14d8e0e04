"""bf16 K/V decode attention and the LSE merge of attention partials (gfx950).

* ``flash_attn_with_kvcache_compat`` mirrors
  ``Z/attn_hub/flash_attn_compat.py:44-100``: q [bs, 1, hq, 128], k_cache /
  v_cache [bs, n, kv, 128] bf16 (any strides with a contiguous last dim, e.g.
  the ``concat.transpose(1, 2)`` views of S:1740-1747), GQA, non-causal (for one
  query token, causal and non-causal agree).  ``softmax_scale`` and
  ``return_softmax_lse`` follow flash_attn_with_kvcache; other keyword
  arguments of that function are not supported and raise.
* ``lse_merge`` / ``lse_merge_torch`` / ``lse_merge_cuda`` mirror
  ``Z/cache_hub/lse_merge/lse_merge.py:79-149``: two outputs [bs, 1, heads, dim]
  with LSEs in [bs, heads, 1], [bs, 1, heads] or [bs, heads].
"""
from __future__ import annotations

import math

import torch

from ._lib import check, device_stream, lib, ptr, require_gpu, stream_of

HEAD_DIM = 128
_WS: dict = {}


def _workspace(device, nbytes: int) -> torch.Tensor:
    """Split partials and arrival slots per (device, stream): calls that may
    overlap on the device (two streams) never share one."""
    dev = torch.device(device)
    key = (dev, device_stream(dev))
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=dev)
        _WS[key] = ws
    return ws


def _check_out(out: torch.Tensor | None, q: torch.Tensor, bs: int, hq: int) -> torch.Tensor:
    """The caller's output buffer ([bs, 1, hq, 128], contiguous, q's dtype or
    float32 for an unrounded result), or a new one in q's dtype."""
    if out is None:
        return torch.empty(bs, 1, hq, HEAD_DIM, dtype=q.dtype, device=q.device)
    if out.dtype not in (q.dtype, torch.float32) or not out.is_contiguous() or out.numel() != bs * hq * HEAD_DIM \
            or out.device != q.device:
        raise ValueError("out must be a contiguous [bs, 1, hq, 128] tensor of q's dtype or float32 on q's device")
    return out


def flash_attn_with_kvcache_compat(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                   causal: bool = False, softmax_scale: float | None = None,
                                   return_softmax_lse: bool = False, out: torch.Tensor | None = None,
                                   n_splits: int = 0, **kwargs):
    """softmax(q K^T * scale) V for one query token per sequence.

    Returns out [bs, 1, hq, 128] in q's dtype (bf16; a float32 ``out`` buffer
    receives the unrounded result), and with ``return_softmax_lse`` also the
    fp32 LSE [bs, hq, 1].  K and V enter the matrix cores as stored (bf16),
    so every finite bf16 value is supported.
    """
    if kwargs:
        raise NotImplementedError(f"flash_attn_with_kvcache_compat: unsupported arguments {sorted(kwargs)}")
    require_gpu(q, k_cache, v_cache)
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("q, k_cache and v_cache must be bfloat16")
    if q.dim() != 4 or q.shape[1] != 1 or q.shape[-1] != HEAD_DIM:
        raise ValueError(f"q must be [bs, 1, hq, 128]; got {tuple(q.shape)}")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.shape[-1] != HEAD_DIM:
        raise ValueError(f"k_cache / v_cache must be [bs, n, kv, 128]; got {tuple(k_cache.shape)}, "
                         f"{tuple(v_cache.shape)}")
    bs, _, hq, _ = q.shape
    kbs, n, kv, _ = k_cache.shape
    if kbs != bs or hq % kv != 0:
        raise ValueError(f"q {tuple(q.shape)} does not match k_cache {tuple(k_cache.shape)}")
    q3 = q[:, 0]
    if q3.stride(-1) != 1 or q3.stride(1) % 8 or q3.stride(0) % 8 or q3.data_ptr() % 16:
        q3 = q3.contiguous()
    if k_cache.stride(-1) != 1 or any(s % 8 for s in k_cache.stride()[:3]) or k_cache.data_ptr() % 16:
        k_cache = k_cache.contiguous()
    if v_cache.stride(-1) != 1 or any(s % 8 for s in v_cache.stride()[:3]) or v_cache.data_ptr() % 16:
        v_cache = v_cache.contiguous()
    scale = 1.0 / math.sqrt(HEAD_DIM) if softmax_scale is None else float(softmax_scale)
    out = _check_out(out, q, bs, hq)
    lse = torch.empty(bs, hq, 1, dtype=torch.float32, device=q.device) if return_softmax_lse else None
    L = lib()
    ws = _workspace(q.device, L.zkv_bf16_attention_workspace_size(bs, hq, kv, n, n_splits))
    check(L.zkv_bf16_decode_attention(
        ptr(q3), q3.stride(0), q3.stride(1),
        ptr(k_cache), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        ptr(v_cache), v_cache.stride(0), v_cache.stride(1), v_cache.stride(2),
        bs, hq, kv, n, scale, ptr(out), int(out.dtype == torch.float32), ptr(lse), n_splits, ptr(ws),
        ws.numel(), stream_of(q)))
    return (out, lse) if return_softmax_lse else out


def gather_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, idx: torch.Tensor | None,
                     tail_start: int = 0, tail_len: int = 0, softmax_scale: float | None = None,
                     return_softmax_lse: bool = False, out: torch.Tensor | None = None,
                     n_splits: int = 0):
    """Decode attention over rows of a bf16 buffer without materialising the
    gather: for (b, kv), the rows idx[b, kv, :] (rows outside the buffer are
    masked out) followed by the contiguous rows [tail_start, tail_start +
    tail_len).  q [bs, 1, hq, 128] bf16; k, v [bs, kv, n_rows, 128] bf16 (any
    strides, rows 16-byte aligned); idx int64 [bs, kv, n_idx] or None.
    Equivalent to gathering those rows, concatenating and calling
    flash_attn_with_kvcache_compat (S:1723-1772)."""
    require_gpu(q, k, v)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("q, k and v must be bfloat16")
    if q.dim() != 4 or q.shape[1] != 1 or q.shape[-1] != HEAD_DIM:
        raise ValueError(f"q must be [bs, 1, hq, 128]; got {tuple(q.shape)}")
    if k.dim() != 4 or k.shape != v.shape or k.shape[-1] != HEAD_DIM:
        raise ValueError(f"k / v must be [bs, kv, n_rows, 128]; got {tuple(k.shape)}, {tuple(v.shape)}")
    bs, _, hq, _ = q.shape
    kbs, kv, n_rows, _ = k.shape
    if kbs != bs or hq % kv != 0:
        raise ValueError(f"q {tuple(q.shape)} does not match k {tuple(k.shape)}")
    for t in (k, v):
        if t.stride(-1) != 1 or any(st % 8 for st in t.stride()[:3]) or t.data_ptr() % 16:
            raise ValueError("k / v rows must be 16-byte aligned with a contiguous last dim")
    n_idx = 0 if idx is None else idx.shape[-1]
    if idx is not None:
        if idx.dtype != torch.int64 or idx.dim() != 3 or tuple(idx.shape[:2]) != (bs, kv):
            raise ValueError("idx must be int64 [bs, kv, n_idx]")
        if n_idx > 1 and idx.stride(2) != 1:
            idx = idx.contiguous()
    q3 = q[:, 0]
    if q3.stride(-1) != 1 or q3.stride(1) % 8 or q3.stride(0) % 8 or q3.data_ptr() % 16:
        q3 = q3.contiguous()
    scale = 1.0 / math.sqrt(HEAD_DIM) if softmax_scale is None else float(softmax_scale)
    out = _check_out(out, q, bs, hq)
    lse = torch.empty(bs, hq, 1, dtype=torch.float32, device=q.device) if return_softmax_lse else None
    L = lib()
    ws = _workspace(q.device, L.zkv_bf16_attention_workspace_size(bs, hq, kv, n_idx + tail_len, n_splits))
    check(L.zkv_bf16_gather_attention(
        ptr(q3), q3.stride(0), q3.stride(1),
        ptr(k), k.stride(0), k.stride(2), k.stride(1), ptr(v), v.stride(0), v.stride(2), v.stride(1),
        n_rows, ptr(idx), idx.stride(0) if idx is not None else 0, idx.stride(1) if idx is not None else 0,
        n_idx, int(tail_start), int(tail_len), bs, hq, kv, scale, ptr(out), int(out.dtype == torch.float32),
        ptr(lse), n_splits,
        ptr(ws), ws.numel(), stream_of(q)))
    return (out, lse) if return_softmax_lse else out


def _canonical_lse(lse: torch.Tensor, attn_out: torch.Tensor) -> torch.Tensor:
    """LSE as [bs, heads] (accepts [bs, heads, 1], [bs, 1, heads], [bs, heads]),
    the shapes lse_merge.py:55-76 accepts."""
    if attn_out.dim() != 4 or attn_out.size(1) != 1:
        raise ValueError(f"attn_out must be [bs, 1, heads, dim], got {tuple(attn_out.shape)}")
    bs, heads = attn_out.size(0), attn_out.size(2)
    if lse.shape == (bs, heads):
        return lse
    if lse.shape == (bs, heads, 1):
        return lse[..., 0]
    if lse.shape == (bs, 1, heads):
        return lse[:, 0]
    raise ValueError("lse must have shape [bs, heads, 1], [bs, 1, heads], or [bs, heads]; "
                     f"got {tuple(lse.shape)} for attn_out={tuple(attn_out.shape)}")


_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def lse_merge(attn_out_a: torch.Tensor, lse_a: torch.Tensor, attn_out_b: torch.Tensor,
              lse_b: torch.Tensor) -> torch.Tensor:
    """Attention over the union of two KV segments from their normalised
    outputs and LSEs; returns [bs, 1, heads, dim] in attn_out_a's dtype."""
    if attn_out_a.shape != attn_out_b.shape:
        raise ValueError(f"attn outputs must have identical shape, got {attn_out_a.shape} and {attn_out_b.shape}")
    if attn_out_a.device != attn_out_b.device:
        raise ValueError("attn outputs must be on the same device")
    require_gpu(attn_out_a, attn_out_b, lse_a, lse_b)
    if attn_out_a.dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {attn_out_a.dtype}")
    la = _canonical_lse(lse_a, attn_out_a).to(torch.float32).contiguous()
    lb = _canonical_lse(lse_b, attn_out_b).to(torch.float32).contiguous()
    a = attn_out_a.contiguous()
    b = attn_out_b.to(a.dtype).contiguous()
    out = torch.empty_like(a)
    bs, _, heads, dim = a.shape
    check(lib().zkv_lse_merge(ptr(a), ptr(la), ptr(b), ptr(lb), ptr(out), _DTYPES[a.dtype], bs, heads,
                              dim, stream_of(a)))
    return out


lse_merge_torch = lse_merge   # the reference's two entry points, one native implementation
lse_merge_cuda = lse_merge
