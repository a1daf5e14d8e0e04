"""Quest page scoring over the gfx950 C ABI.

Mirrors the reference's loader API: ``load_kernel_module()`` returns an object
whose ``quest_chunk_score(q, chunk_min, chunk_max, scores, n_chunks, valid)``
has the signature of the CUDA extension (Z/cache_hub/quest/quest_chunk_score.cu:536-540,
loaded by Z/cache_hub/quest/quest_ops.py:89-107).  There is no PyTorch
fallback: a missing library raises.
"""
from __future__ import annotations

import torch

from ._lib import check, device_stream, lib, ptr, require_gpu, stream_of


def quest_chunk_score(q: torch.Tensor, chunk_min: torch.Tensor, chunk_max: torch.Tensor,
                      scores: torch.Tensor, n_chunks: int, valid: torch.Tensor | None = None) -> None:
    """scores[b, h, c] = sum_d max(q_d mn_d, q_d mx_d) for c < n_chunks, in place.

    q bf16 [bs, kv, 128]; chunk_min / chunk_max [bs, kv, n_max, 128] bf16 (the
    reference) or fp16; scores fp32 [bs, kv, n_chunks]; valid bool
    [bs, kv, n_max] or None (invalid chunks score -inf).
    """
    require_gpu(q, chunk_min, chunk_max, scores)
    if q.dtype != torch.bfloat16:
        raise RuntimeError(f"quest_chunk_score: only bf16 q is supported; got {q.dtype}")
    if chunk_min.dtype != chunk_max.dtype or chunk_min.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("quest_chunk_score: chunk_min / chunk_max must both be bf16 or fp16")
    bs, kv, d = q.shape
    if d != 128:
        raise RuntimeError(f"quest_chunk_score: only head_dim==128 is supported; got {d}")
    n_max = chunk_min.shape[2]
    n_chunks = int(n_chunks)
    if n_chunks > n_max:
        raise RuntimeError("n_chunks must <= chunk_n_max")
    for name, t in (("q", q), ("chunk_min", chunk_min), ("chunk_max", chunk_max), ("scores", scores)):
        if not t.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")
    if tuple(chunk_min.shape) != (bs, kv, n_max, 128) or chunk_max.shape != chunk_min.shape:
        raise RuntimeError("chunk_min / chunk_max must be [bs, kv, n_chunks_max, 128]")
    if scores.dtype != torch.float32 or scores.numel() != bs * kv * n_chunks:
        raise RuntimeError("scores must be fp32 [bs, kv, n_chunks]")
    if valid is not None:
        if valid.dtype != torch.bool or not valid.is_contiguous() or tuple(valid.shape) != (bs, kv, n_max):
            raise RuntimeError("valid must be a contiguous bool [bs, kv, n_chunks_max]")
    check(lib().zkv_quest_chunk_score(
        ptr(q), ptr(chunk_min), ptr(chunk_max), int(chunk_min.dtype == torch.float16), ptr(scores),
        bs, kv, n_chunks, n_max, ptr(valid), stream_of(q)))


def page_minmax_f16(keys: torch.Tensor, page_size: int = 16, n_pages: int | None = None,
                    page_min: torch.Tensor | None = None, page_max: torch.Tensor | None = None):
    """Per-page fp16 (min rounded down, max rounded up) of bf16 keys
    [bs, kv, n_tok, 128] (any strides with a contiguous last dim).

    Returns (page_min, page_max) fp16 [bs, kv, n_pages_max, 128]; pages
    [0, n_pages) are written (default n_tok // page_size).
    """
    require_gpu(keys)
    if keys.dtype != torch.bfloat16 or keys.dim() != 4 or keys.shape[-1] != 128 or keys.stride(-1) != 1:
        raise RuntimeError("keys must be bf16 [bs, kv, n_tok, 128] with a contiguous last dim")
    bs, kv, n_tok, _ = keys.shape
    n_pages = n_tok // page_size if n_pages is None else int(n_pages)
    if n_pages * page_size > n_tok:
        raise RuntimeError(f"{n_pages} pages of {page_size} exceed {n_tok} tokens")
    if page_min is None:
        page_min = torch.empty(bs, kv, n_pages, 128, dtype=torch.float16, device=keys.device)
    if page_max is None:
        page_max = torch.empty_like(page_min)
    for t in (page_min, page_max):
        if t.dtype != torch.float16 or not t.is_contiguous() or t.shape[:2] != (bs, kv) or t.shape[3] != 128:
            raise RuntimeError("page_min / page_max must be contiguous fp16 [bs, kv, n_pages_max, 128]")
    n_max = page_min.shape[2]
    check(lib().zkv_page_minmax_f16(ptr(keys), keys.stride(0), keys.stride(1), keys.stride(2), bs, kv,
                                    page_size, n_pages, n_max, ptr(page_min), ptr(page_max),
                                    stream_of(keys)))
    return page_min, page_max


def quest_chunk_score_gqa(queries: torch.Tensor, kv_heads: int, chunk_min: torch.Tensor,
                          chunk_max: torch.Tensor, scores: torch.Tensor, n_chunks: int,
                          valid: torch.Tensor | None, raw_q: torch.Tensor) -> torch.Tensor:
    """GQA-mean query (S:1621-1626) and Quest bounds in one launch.

    queries bf16 [bs, hq, 128] or [bs, 1, hq, 128] (last dim contiguous);
    raw_q bf16 [bs, kv, 128] contiguous receives bf16(mean over each KV
    head's query heads), the query the bounds are scored with.  The other
    arguments are those of ``quest_chunk_score``.  Returns raw_q.
    """
    q = queries.reshape(queries.shape[0], -1, queries.shape[-1]) if queries.dim() == 4 else queries
    require_gpu(q, chunk_min, chunk_max, scores, raw_q)
    if q.dtype != torch.bfloat16 or raw_q.dtype != torch.bfloat16:
        raise RuntimeError("quest_chunk_score_gqa: queries and raw_q must be bf16")
    bs, hq, d = q.shape
    if d != 128 or q.stride(-1) != 1:
        raise RuntimeError("quest_chunk_score_gqa: queries need head_dim 128, contiguous")
    kv = int(kv_heads)
    if hq % kv or raw_q.shape != (bs, kv, 128) or not raw_q.is_contiguous():
        raise RuntimeError("quest_chunk_score_gqa: raw_q must be a contiguous [bs, kv, 128] with kv | hq")
    if chunk_min.dtype != chunk_max.dtype or chunk_min.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("quest_chunk_score_gqa: chunk_min / chunk_max must both be bf16 or fp16")
    n_max = chunk_min.shape[2]
    n_chunks = int(n_chunks)
    if not 1 <= n_chunks <= n_max:
        raise RuntimeError("quest_chunk_score_gqa: need 1 <= n_chunks <= chunk_n_max")
    if chunk_min.shape != (bs, kv, n_max, 128) or chunk_max.shape != chunk_min.shape \
            or not chunk_min.is_contiguous() or not chunk_max.is_contiguous():
        raise RuntimeError("chunk_min / chunk_max must be contiguous [bs, kv, n_chunks_max, 128]")
    if scores.dtype != torch.float32 or scores.numel() != bs * kv * n_chunks or not scores.is_contiguous():
        raise RuntimeError("scores must be fp32 [bs, kv, n_chunks]")
    if valid is not None:
        if valid.dtype != torch.bool or not valid.is_contiguous() or tuple(valid.shape) != (bs, kv, n_max):
            raise RuntimeError("valid must be a contiguous bool [bs, kv, n_chunks_max]")
    check(lib().zkv_quest_chunk_score_gqa(
        ptr(q), q.stride(0), q.stride(1), hq, ptr(raw_q), ptr(chunk_min), ptr(chunk_max),
        int(chunk_min.dtype == torch.float16), ptr(scores), bs, kv, n_chunks, n_max, ptr(valid),
        stream_of(q)))
    return raw_q


QUEST_TOPK_MAX_CHUNKS = 4096     # rows the fused scan + top-k launch takes
_SLOTS: dict = {}


def _slots(device: torch.device, n: int) -> torch.Tensor:
    """Arrival counters of the fused launch per (device, stream): zeroed when
    made, left zero by every launch; concurrent launches never share one."""
    key = (device, device_stream(device))
    t = _SLOTS.get(key)
    if t is None or t.numel() < n:
        t = torch.zeros(max(n, 256), dtype=torch.int32, device=device)
        _SLOTS[key] = t
    return t


def quest_chunk_topk_gqa(queries: torch.Tensor, kv_heads: int, chunk_min: torch.Tensor,
                         chunk_max: torch.Tensor, scores: torch.Tensor, n_chunks: int,
                         valid: torch.Tensor | None, raw_q: torch.Tensor, k: int,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """``quest_chunk_score_gqa`` and ``float_topk_3d(scores, k)`` in one launch:
    GQA-mean query, Quest bounds (written to ``scores``, the same bits) and the
    top-k chunk indices of every (b, kv) row, int64 [bs, kv, k] in increasing
    index order (the same indices as float_topk_3d; -1 past n_chunks when
    k > n_chunks).  Rows of up to 4096 chunks.  ``out`` (optional, int64
    [bs, kv, >= k] with a contiguous last dim) receives the indices; returns
    them."""
    args, q, ret, _ = _quest_topk_args(queries, kv_heads, chunk_min, chunk_max, scores, n_chunks, valid, raw_q,
                                       k, out)
    check(lib().zkv_quest_chunk_topk_gqa(*args, stream_of(q)))
    return ret


class QuestTopkPlan:
    """``quest_chunk_topk_gqa`` with its checks done once for fixed buffers (a
    decode loop: new query and metadata contents, the same tensors): ``run()``
    is one C-ABI call on the current stream and returns the indices.  The
    tensors must stay alive and keep their shapes and strides; the arrival
    counters are the ones cached for the stream current at creation, so run
    the plan on that stream."""

    def __init__(self, queries, kv_heads, chunk_min, chunk_max, scores, n_chunks, valid, raw_q, k, out=None):
        self._args, self._q, self.out, self._keep = _quest_topk_args(queries, kv_heads, chunk_min, chunk_max,
                                                                     scores, n_chunks, valid, raw_q, k, out)
        self._fn = lib().zkv_quest_chunk_topk_gqa

    def run(self) -> torch.Tensor:
        check(self._fn(*self._args, stream_of(self._q)))
        return self.out


def _quest_topk_args(queries, kv_heads, chunk_min, chunk_max, scores, n_chunks, valid, raw_q, k, out):
    """Checked arguments of zkv_quest_chunk_topk_gqa (all but the stream), the
    query view, the indices to return and the tensors the pointers belong to."""
    q = queries.reshape(queries.shape[0], -1, queries.shape[-1]) if queries.dim() == 4 else queries
    require_gpu(q, chunk_min, chunk_max, scores, raw_q)
    bs, hq, _ = q.shape
    kv = int(kv_heads)
    n_max = chunk_min.shape[2]
    n_chunks, k = int(n_chunks), int(k)
    if not 1 <= n_chunks <= min(n_max, QUEST_TOPK_MAX_CHUNKS):
        raise RuntimeError(f"quest_chunk_topk_gqa: n_chunks={n_chunks} outside [1, {min(n_max, QUEST_TOPK_MAX_CHUNKS)}]")
    if not 1 <= k:
        raise RuntimeError(f"quest_chunk_topk_gqa: k={k}")
    # the shape / dtype checks of quest_chunk_score_gqa
    if q.dtype != torch.bfloat16 or raw_q.dtype != torch.bfloat16 or q.shape[-1] != 128 or q.stride(-1) != 1:
        raise RuntimeError("quest_chunk_topk_gqa: queries and raw_q must be bf16 with head_dim 128")
    if hq % kv or raw_q.shape != (bs, kv, 128) or not raw_q.is_contiguous():
        raise RuntimeError("quest_chunk_topk_gqa: raw_q must be a contiguous [bs, kv, 128] with kv | hq")
    if chunk_min.dtype != chunk_max.dtype or chunk_min.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError("quest_chunk_topk_gqa: chunk_min / chunk_max must both be bf16 or fp16")
    if chunk_min.shape != (bs, kv, n_max, 128) or chunk_max.shape != chunk_min.shape \
            or not chunk_min.is_contiguous() or not chunk_max.is_contiguous():
        raise RuntimeError("chunk_min / chunk_max must be contiguous [bs, kv, n_chunks_max, 128]")
    if scores.dtype != torch.float32 or scores.numel() != bs * kv * n_chunks or not scores.is_contiguous():
        raise RuntimeError("scores must be fp32 [bs, kv, n_chunks]")
    if valid is not None:
        if valid.dtype != torch.bool or not valid.is_contiguous() or tuple(valid.shape) != (bs, kv, n_max):
            raise RuntimeError("valid must be a contiguous bool [bs, kv, n_chunks_max]")
    if out is None:
        out = torch.empty(bs, kv, k, dtype=torch.int64, device=q.device)
    elif out.dtype != torch.int64 or out.shape[0] != bs or out.shape[1] != kv or out.shape[2] < k or out.stride(2) != 1 \
            or out.stride(0) != kv * out.stride(1):
        raise RuntimeError("out must be int64 [bs, kv, >= k] with rows at one stride")
    sl = _slots(q.device, bs * kv)
    args = (ptr(q), q.stride(0), q.stride(1), hq, ptr(raw_q), ptr(chunk_min), ptr(chunk_max),
            int(chunk_min.dtype == torch.float16), ptr(scores), bs, kv, n_chunks, n_max, ptr(valid), k,
            ptr(out), out.stride(1), ptr(sl), sl.numel() * 4)
    owners = (q, chunk_min, chunk_max, scores, valid, raw_q, out, sl)
    return args, q, (out if out.shape[2] == k else out[:, :, :k]), owners


class QuestKernel:
    """Drop-in for the module ``quest_ops.load_kernel_module()`` returns."""

    @staticmethod
    def quest_chunk_score(q, chunk_min, chunk_max, scores, n_chunks, valid=None):
        quest_chunk_score(q, chunk_min, chunk_max, scores, n_chunks, valid)


def load_kernel_module() -> QuestKernel:
    lib()  # fail loudly now if the native library is missing
    return QuestKernel()
