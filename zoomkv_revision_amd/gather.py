"""Host-to-device gather of bf16 K / V rows from pinned host memory
(the reference's ``cache_hub.gather_trans.trans_h2d``, trans_h2d.py:65-166).

The kernels read the selected rows of pinned host buffers through their
device alias, so only those rows cross the host link.  Same names, argument
order and assertions as the reference's wrappers; the ``load_kernel_module``
JIT step is replaced by the prebuilt library.
"""
from __future__ import annotations

import torch

from ._lib import check, lib, ptr, stream_of


def h2d_gather_kv(src_k_caches, src_v_caches, selected_indices, dst_k_caches, dst_v_caches) -> None:
    """dst[b, h, j] = src[b, h, selected_indices[b, h, j]] for j < topk
    (trans_h2d.py:65-103).  src: pinned CPU [bs, heads, kv_len, 128] bf16;
    indices / dst on the GPU; dst [bs, heads, >= topk, 128].  An index outside
    [0, kv_len) leaves its destination row untouched."""
    bs, heads, kv_len, dim = src_k_caches.shape
    assert src_k_caches.shape == src_v_caches.shape
    _, _, topk = selected_indices.shape
    assert dst_k_caches.shape == dst_v_caches.shape
    assert dst_k_caches.shape[-2] >= topk
    assert dim == 128
    assert src_k_caches.is_cpu and src_v_caches.is_cpu
    assert src_k_caches.is_pinned() and src_v_caches.is_pinned()
    assert dst_k_caches.is_cuda and dst_v_caches.is_cuda
    assert src_k_caches.dtype == src_v_caches.dtype
    assert dst_k_caches.dtype == dst_v_caches.dtype
    assert src_k_caches.dtype == dst_k_caches.dtype
    assert src_k_caches.dtype == torch.bfloat16
    assert src_k_caches.is_contiguous() and dst_k_caches.is_contiguous()
    assert src_v_caches.is_contiguous() and dst_v_caches.is_contiguous()
    assert tuple(dst_k_caches.shape[:2]) == (bs, heads) and tuple(selected_indices.shape[:2]) == (bs, heads)
    idx = selected_indices
    if idx.dtype != torch.int64 or not idx.is_contiguous() or idx.device != dst_k_caches.device:
        idx = idx.to(device=dst_k_caches.device, dtype=torch.int64).contiguous()
    check(lib().zkv_h2d_gather_kv(ptr(src_k_caches), ptr(src_v_caches), bs, heads, kv_len, ptr(idx), topk,
                                  ptr(dst_k_caches), ptr(dst_v_caches), dst_k_caches.shape[2],
                                  stream_of(dst_k_caches)))


def h2d_gather_kv_packed(src_k_caches, src_v_caches, dst_k_packed, dst_v_packed, indices_packed,
                         cu_seqlens_topk, cu_seqlens_k, sl_end: int, global_k: int) -> None:
    """Variable-K gather into the packed varlen buffers (trans_h2d.py:106-166):
    segment vh = b * kv_heads + h writes rows [cu_seqlens_k[vh] + sl_end,
    ...) with the indices indices_packed[cu_seqlens_topk[vh] ..
    cu_seqlens_topk[vh + 1]); the first sl_end rows of a segment are the
    caller's."""
    bs, kv_heads, src_len, dim = src_k_caches.shape
    V = bs * kv_heads
    assert src_k_caches.shape == src_v_caches.shape
    assert dim == 128
    assert src_k_caches.is_cpu and src_v_caches.is_cpu
    assert src_k_caches.is_pinned() and src_v_caches.is_pinned()
    assert dst_k_packed.is_cuda and dst_v_packed.is_cuda
    assert indices_packed.is_cuda
    assert cu_seqlens_topk.is_cuda and cu_seqlens_k.is_cuda
    assert src_k_caches.dtype == torch.bfloat16 and src_v_caches.dtype == torch.bfloat16
    assert dst_k_packed.dtype == torch.bfloat16 and dst_v_packed.dtype == torch.bfloat16
    assert indices_packed.dtype == torch.int64
    assert cu_seqlens_topk.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32
    assert src_k_caches.is_contiguous() and src_v_caches.is_contiguous()
    assert dst_k_packed.is_contiguous() and dst_v_packed.is_contiguous()
    assert dst_k_packed.dim() == 2 and dst_k_packed.shape[1] == dim
    assert dst_v_packed.shape == dst_k_packed.shape
    assert cu_seqlens_topk.shape[0] == V + 1
    assert cu_seqlens_k.shape[0] == V + 1
    assert indices_packed.dim() == 1
    check(lib().zkv_h2d_gather_kv_packed(
        ptr(src_k_caches), ptr(src_v_caches), bs, kv_heads, src_len, ptr(dst_k_packed), ptr(dst_v_packed),
        dst_k_packed.shape[0], ptr(indices_packed.contiguous()), indices_packed.numel(),
        ptr(cu_seqlens_topk.contiguous()), ptr(cu_seqlens_k.contiguous()), int(sl_end), int(global_k),
        stream_of(dst_k_packed)))
