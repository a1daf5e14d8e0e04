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


def copy_rows(dst: torch.Tensor, src: torch.Tensor) -> None:
    """dst.copy_(src) for [rows, n, 128]-shaped views whose last two dims are
    contiguous (any row stride), as one pitched copy on the current stream:
    device and pinned host memory on either side, asynchronous like
    ``copy_(..., non_blocking=True)`` (the flush's D2H move, S:1465-1469)."""
    assert dst.dtype == src.dtype and dst.shape == src.shape, "copy_rows: shape / dtype mismatch"
    assert dst.dim() >= 2 and src.dim() >= 2
    for t in (dst, src):
        assert t.stride(-1) == 1 and t.stride(-2) == t.shape[-1], "copy_rows: the last two dims must be contiguous"
        assert t.is_cuda or t.is_pinned(), "copy_rows: host memory must be pinned"
        # the leading dims must collapse to one row index with a single pitch
        lead = t.shape[:-2]
        for i in range(len(lead) - 1):
            assert t.stride(i) == t.stride(i + 1) * lead[i + 1], "copy_rows: leading dims must collapse"
    row_bytes = src.shape[-2] * src.shape[-1] * src.element_size()
    rows = src.numel() // (src.shape[-2] * src.shape[-1]) if src.numel() else 0
    pitch = lambda t: (t.stride(-3) if t.dim() >= 3 else t.shape[-2] * t.shape[-1]) * t.element_size()
    dev = dst if dst.is_cuda else src
    check(lib().zkv_copy_rows(ptr(dst), pitch(dst), ptr(src), pitch(src), row_bytes, rows, stream_of(dev)))


def pinned_empty(shape, dtype: torch.dtype) -> torch.Tensor:
    """An uninitialised pinned host tensor of exactly its size (the library's
    hipHostMalloc; torch's pinned allocator rounds each block up to a power of
    two).  The memory is released when the last tensor viewing it is gone."""
    import ctypes as C
    n = 1
    for s in shape:
        n *= int(s)
    nbytes = max(n * torch.empty(0, dtype=dtype).element_size(), 1)
    p = C.c_void_p()
    check(lib().zkv_host_alloc(nbytes, C.byref(p)))
    free, addr = lib().zkv_host_free, p.value
    # the ctypes block owns the allocation: torch.frombuffer keeps it alive
    # for as long as any view of the storage exists
    block = type("PinnedBlock", (C.c_uint8 * nbytes,), {"__del__": lambda self: free(addr)})
    buf = block.from_address(addr)
    return torch.frombuffer(buf, dtype=torch.uint8)[:n * torch.empty(0, dtype=dtype).element_size()] \
        .view(dtype).view(*shape)
