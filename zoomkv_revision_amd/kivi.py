"""Host side of the KIVI 4-bit cache: Format R chunk encode, Format Q pack and
the fused 4-bit decode attention, over the gfx950 C ABI.

Format R is the reference's K cache (S:646-744); ``chunk_encode`` replaces the
aligned-chunk branch of ``_compute_and_store_chunk_minmax`` +
``_kivi_pack_chunks`` (S:2119-2143, S:1965-2020).  Format Q is the north-star
K+V cache with fp16 scale/zero (no reference counterpart; V is bf16 in the
reference, S:561-571).
"""
from __future__ import annotations

import functools
import math
from dataclasses import dataclass

import torch

from ._lib import check, device_stream, lib, ptr, require_gpu, stream_of

HEAD_DIM = 128
GROUP = 32  # Format Q tokens per group


def _check_bf16(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16; got {t.dtype}")


def _check_last_contig(name: str, t: torch.Tensor) -> None:
    if t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous last dim of {HEAD_DIM}; "
                         f"got shape {tuple(t.shape)} stride {t.stride()}")


# ---------------------------------------------------------------------------
# Format R
# ---------------------------------------------------------------------------
def chunk_encode(keys: torch.Tensor, chunk_size: int, chunk_start: int,
                 chunk_min: torch.Tensor, chunk_max: torch.Tensor,
                 chunk_centroid: torch.Tensor, chunk_valid: torch.Tensor,
                 packed_K: torch.Tensor) -> int:
    """Encode the ``keys.shape[2] // chunk_size`` full chunks of ``keys``.

    keys [bs, kv, n_tok, 128] bf16 (any token / head / batch stride);
    chunk_min/max/centroid [bs, kv, n_chunks_max, 128] bf16 contiguous;
    chunk_valid [bs, kv, n_chunks_max] bool; packed_K [bs, kv, n_chunks_max,
    16, chunk_size] int32 contiguous.  Writes chunks [chunk_start,
    chunk_start + n) in place and returns n.
    """
    require_gpu(keys, chunk_min, chunk_max, chunk_centroid, chunk_valid, packed_K)
    _check_bf16("keys", keys)
    _check_last_contig("keys", keys)
    for n, t in (("chunk_min", chunk_min), ("chunk_max", chunk_max), ("chunk_centroid", chunk_centroid)):
        _check_bf16(n, t)
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    if chunk_valid.dtype != torch.bool or packed_K.dtype != torch.int32:
        raise TypeError("chunk_valid must be bool and packed_K int32")
    bs, kv, n_tok, _ = keys.shape
    n_max = chunk_min.shape[2]
    if tuple(packed_K.shape) != (bs, kv, n_max, 16, chunk_size) or not packed_K.is_contiguous():
        raise ValueError(f"packed_K must be contiguous [{bs}, {kv}, {n_max}, 16, {chunk_size}]; "
                         f"got {tuple(packed_K.shape)}")
    n = n_tok // chunk_size
    check(lib().zkv_chunk_encode(
        ptr(keys), keys.stride(0), keys.stride(1), keys.stride(2), bs, kv, chunk_size, n,
        chunk_start, n_max, ptr(chunk_min), ptr(chunk_max), ptr(chunk_centroid),
        ptr(chunk_valid), ptr(packed_K), stream_of(keys)))
    return n


# ---------------------------------------------------------------------------
# Format Q
# ---------------------------------------------------------------------------
RECORD_WORDS = 1280   # one 32-token group of one KV head: 5120 bytes


@dataclass
class Kivi4Cache:
    """Device storage of a Format Q cache plus its bf16 residual window.

    ``groups`` int32 [bs, kv, G_cap, 1280] holds one contiguous 5120-byte
    record per 32-token group: K codes (words 0-511), V codes (512-1023),
    K scale/zero (1024-1151) and V scale/zero (1152-1279), each in the decode
    kernel's MFMA operand order; the codes and V scale/zero of each 16-token
    half (one Quest page) are separate blocks.  ``k_codes`` / ``v_codes`` /
    ``k_meta`` / ``v_meta`` are views of those parts."""
    groups: torch.Tensor    # int32 [bs, kv, G_cap, 1280]
    k_res: torch.Tensor     # bf16  [bs, kv, R_cap, 128]
    v_res: torch.Tensor     # bf16  [bs, kv, R_cap, 128]
    n_groups: int = 0
    res_len: int = 0

    @classmethod
    def allocate(cls, bs: int, kv: int, g_cap: int, r_cap: int = 128,
                 device: torch.device | str = "cuda") -> "Kivi4Cache":
        z = dict(device=device)
        return cls(
            torch.zeros(bs, kv, g_cap, RECORD_WORDS, dtype=torch.int32, **z),
            torch.zeros(bs, kv, r_cap, HEAD_DIM, dtype=torch.bfloat16, **z),
            torch.zeros(bs, kv, r_cap, HEAD_DIM, dtype=torch.bfloat16, **z),
        )

    def rows(self, b0: int, b1: int) -> "Kivi4Cache":
        """The cache of batch rows [b0, b1) (views)."""
        return Kivi4Cache(self.groups[b0:b1], self.k_res[b0:b1], self.v_res[b0:b1], self.n_groups,
                          self.res_len)

    @property
    def k_codes(self) -> torch.Tensor:   # int32 [bs, kv, G_cap, 512]
        return self.groups[..., 0:512]

    @property
    def v_codes(self) -> torch.Tensor:   # int32 [bs, kv, G_cap, 512]
        return self.groups[..., 512:1024]

    @property
    def k_meta(self) -> torch.Tensor:    # fp16 [bs, kv, G_cap, 16, 2, 8]
        return self.groups[..., 1024:1152].view(torch.float16).unflatten(-1, (16, 2, 8))

    @property
    def v_meta(self) -> torch.Tensor:    # fp16 [bs, kv, G_cap, 2, 4, 4, 2, 4]
        return self.groups[..., 1152:1280].view(torch.float16).unflatten(-1, (2, 4, 4, 2, 4))

    @property
    def g_cap(self) -> int:
        return self.groups.shape[2]

    @property
    def r_cap(self) -> int:
        return self.k_res.shape[2]

    @property
    def shape(self):
        return self.groups.shape[0], self.groups.shape[1]

    def nbytes_per_token(self) -> int:
        return 160  # K codes 64 + K meta 16 + V codes 64 + V meta 16


_RANGE_STATUS: dict = {}
RANGE_K, RANGE_V, RANGE_V_SCALE = 1, 2, 4   # ZKV_RANGE_* bits of the C ABI
_RANGE_MESSAGES = ((RANGE_K, "a K scale or zero point beyond fp16 (|K| > 65504)"),
                   (RANGE_V, "a V scale or zero point beyond fp16 (|V| > 65504)"),
                   (RANGE_V_SCALE, "a V scale above 2048 (V range > 30720 in one 32-channel group)"))


def _range_status(device: torch.device) -> torch.Tensor:
    """The per-device status word that range-checked packs OR their ZKV_RANGE_*
    bits into (zeroed when created and by ``kivi4_pack_status``)."""
    key = (device.type, device.index)
    t = _RANGE_STATUS.get(key)
    if t is None:
        t = torch.zeros(1, dtype=torch.int32, device=device)
        _RANGE_STATUS[key] = t
    return t


def kivi4_pack(k: torch.Tensor, v: torch.Tensor, cache: Kivi4Cache, g0: int,
               check_range: bool = True) -> int:
    """Quantize the leading full groups of k / v [bs, kv, n, 128] into groups
    [g0, g0 + n // 32) of ``cache``; returns the number of groups written.

    The call never synchronises the host.  With ``check_range`` (the default)
    the pack ORs a bit into the device's status word whenever a group's fp16
    scale / zero cannot hold its values (|K| or |V| or a group's range beyond
    65504) or a V scale exceeds the decode kernel's limit of 2048 (a V range
    above 30720 inside one 32-channel group); the caller reads it at its next
    synchronisation point with ``check_kivi4_pack_range`` (raises
    ``RuntimeError``) or ``kivi4_pack_status``.  ``check_range=False`` skips
    the check, for callers that bound their values themselves."""
    require_gpu(k, v)
    _check_bf16("k", k)
    _check_bf16("v", v)
    _check_last_contig("k", k)
    _check_last_contig("v", v)
    if k.shape != v.shape:
        raise ValueError(f"k / v shape mismatch {tuple(k.shape)} vs {tuple(v.shape)}")
    bs, kv, n, _ = k.shape
    if (bs, kv) != tuple(cache.shape):
        raise ValueError("cache batch / head shape mismatch")
    ng = n // GROUP
    status = _range_status(k.device) if check_range else None
    check(lib().zkv_kivi4_pack(
        ptr(k), k.stride(0), k.stride(1), k.stride(2),
        ptr(v), v.stride(0), v.stride(1), v.stride(2),
        bs, kv, ng, g0, cache.g_cap,
        ptr(cache.groups), ptr(status), stream_of(k)))
    return ng


def kivi4_prefill(k: torch.Tensor, v: torch.Tensor, cache: Kivi4Cache, res_len: int,
                  check_range: bool = True) -> tuple[int, int]:
    """Prefill of a Format Q cache in one launch: of the n tokens of k / v
    [bs, kv, n, 128], the first n - res_len (a multiple of 32) are quantized
    into groups [0, (n - res_len) / 32) as ``kivi4_pack`` does, and the last
    ``res_len`` are copied as bf16 rows into rows [0, res_len) of the residual
    window.  Returns (n_groups, res_len), the arguments the decode attention
    takes.  The range check is ``kivi4_pack``'s (asynchronous)."""
    args, ret, _ = _prefill_args(k, v, cache, res_len, check_range)
    check(lib().zkv_kivi4_prefill(*args, stream_of(k)))
    return ret


class PrefillPlan:
    """``kivi4_prefill`` with its checks done once for fixed buffers: ``run()``
    is one C-ABI call on the current stream over the buffers' current
    contents and returns (n_groups, res_len).  The tensors must stay alive
    and keep their shapes and strides."""

    def __init__(self, k, v, cache, res_len, check_range=True):
        self._k = k
        self._args, self.result, self._keep = _prefill_args(k, v, cache, res_len, check_range)
        self._fn = lib().zkv_kivi4_prefill

    def run(self) -> tuple[int, int]:
        check(self._fn(*self._args, stream_of(self._k)))
        return self.result


def _prefill_args(k, v, cache, res_len, check_range):
    """Checked arguments of zkv_kivi4_prefill (all but the stream), the
    result to return and the tensors the pointers belong to."""
    require_gpu(k, v)
    _check_bf16("k", k)
    _check_bf16("v", v)
    _check_last_contig("k", k)
    _check_last_contig("v", v)
    if k.shape != v.shape:
        raise ValueError(f"k / v shape mismatch {tuple(k.shape)} vs {tuple(v.shape)}")
    bs, kv, n, _ = k.shape
    if (bs, kv) != tuple(cache.shape):
        raise ValueError("cache batch / head shape mismatch")
    res_len = int(res_len)
    nq = n - res_len
    if res_len < 0 or nq < 0 or nq % GROUP:
        raise ValueError(f"n - res_len = {nq} must be a non-negative multiple of {GROUP}")
    if res_len > cache.r_cap or nq // GROUP > cache.g_cap:
        raise ValueError("prefill exceeds the cache capacity")
    if not (cache.k_res.is_contiguous() and cache.v_res.is_contiguous()):
        raise ValueError("the residual windows must be contiguous [bs, kv, r_cap, 128]")
    status = _range_status(k.device) if check_range else None
    args = (ptr(k), k.stride(0), k.stride(1), k.stride(2),
            ptr(v), v.stride(0), v.stride(1), v.stride(2),
            bs, kv, nq // GROUP, 0, cache.g_cap, ptr(cache.groups), ptr(status),
            ptr(cache.k_res), ptr(cache.v_res), cache.r_cap, 0, res_len)
    return args, (nq // GROUP, res_len), (k, v, cache.groups, cache.k_res, cache.v_res, status)


def kivi4_pack_status(device: torch.device | str | None = None, clear: bool = True) -> int:
    """The ZKV_RANGE_* bits that range-checked packs on ``device`` (default: the
    current device) recorded since the last clear.  Reading the word waits for
    the packs queued before it on the current stream (a host synchronisation);
    ``clear`` resets it to 0 afterwards, in stream order."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    t = _range_status(dev)
    bits = int(t.item())
    if clear and bits:
        t.zero_()
    return bits


def check_kivi4_pack_range(device: torch.device | str | None = None) -> None:
    """Raise ``RuntimeError`` naming what went out of range if any range-checked
    pack on ``device`` since the last check stored values beyond the 4-bit
    cache's fp16 range (see ``kivi4_pack``); clears the status."""
    bits = kivi4_pack_status(device, clear=True)
    if bits:
        what = [name for bit, name in _RANGE_MESSAGES if bits & bit]
        raise RuntimeError("kivi4_pack: values outside the 4-bit cache's fp16 range: " + "; ".join(what))


_WORKSPACE: dict = {}


@functools.lru_cache(maxsize=256)
def _decode_ws_bytes(bs: int, hq: int, kv: int, n_groups: int, res_len: int, n_splits: int) -> int:
    return lib().zkv_kivi4_attention_workspace_size(bs, hq, kv, n_groups, res_len, n_splits)


@functools.lru_cache(maxsize=256)
def _sparse_ws_bytes(bs: int, hq: int, kv: int, n_sel: int, res_len: int, n_splits: int) -> int:
    return lib().zkv_kivi4_sparse_attention_workspace_size(bs, hq, kv, n_sel, res_len, n_splits)


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Attention workspace (split partials and arrival slots) per (device,
    stream), grown on demand: calls on one stream run in order, and calls on
    two streams, which may overlap on the device, get two workspaces."""
    key = (device.type, device.index, device_stream(device))
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACE[key] = ws
    return ws


def attention_workspace(bs: int, hq: int, kv: int, n_groups: int, res_len: int,
                        n_splits: int = 0, device="cuda") -> torch.Tensor:
    """A dedicated workspace for ``kivi4_decode_attention``."""
    n = lib().zkv_kivi4_attention_workspace_size(bs, hq, kv, n_groups, res_len, n_splits)
    return torch.zeros(n, dtype=torch.uint8, device=device)


def kivi4_decode_attention(q: torch.Tensor, cache: Kivi4Cache, n_groups: int | None = None,
                           res_len: int | None = None, sm_scale: float | None = None,
                           out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                           n_splits: int = 0, workspace: torch.Tensor | None = None,
                           return_lse: bool = False):
    """Decode attention of q [bs, hq, 128] or [bs, 1, hq, 128] (bf16) over the
    first ``n_groups`` groups and ``res_len`` residual tokens of ``cache``.

    Output has q's shape and ``out_dtype`` (default q.dtype; float32 allowed).
    With ``return_lse`` also the fp32 natural-log LSE [bs, hq] of the scaled
    scores (flash-attn's softmax_lse).
    """
    args, ret, _ = _decode_args(q, cache, n_groups, res_len, sm_scale, out, out_dtype, n_splits, workspace,
                                return_lse)
    check(lib().zkv_kivi4_decode_attention(*args, stream_of(q)))
    return ret


class DecodeAttentionPlan:
    """``kivi4_decode_attention`` with its checks done once for fixed buffers
    (a decode loop: new query and cache contents, the same tensors and
    lengths): ``run()`` is one C-ABI call on the current stream and returns
    the output (and LSE).  The tensors must stay alive and keep their shapes
    and strides; without a ``workspace`` the plan takes the one cached for the
    stream current at creation, so run it on that stream."""

    def __init__(self, q, cache, n_groups=None, res_len=None, sm_scale=None, out=None, out_dtype=None, n_splits=0,
                 workspace=None, return_lse=False):
        self._q = q
        self._args, self.out, self._keep = _decode_args(q, cache, n_groups, res_len, sm_scale, out, out_dtype,
                                                        n_splits, workspace, return_lse)
        self._fn = lib().zkv_kivi4_decode_attention

    def run(self):
        check(self._fn(*self._args, stream_of(self._q)))
        return self.out


def _decode_args(q, cache, n_groups, res_len, sm_scale, out, out_dtype, n_splits, workspace, return_lse):
    """Checked arguments of zkv_kivi4_decode_attention (all but the stream),
    the result to return and the tensors the pointers belong to."""
    require_gpu(q)
    _check_bf16("q", q)
    squeeze = False
    if q.dim() == 4:
        if q.shape[1] != 1:
            raise ValueError("decode attention takes one query token per sequence")
        q3 = q[:, 0]
        squeeze = True
    else:
        q3 = q
    _check_last_contig("q", q3)
    bs, hq, _ = q3.shape
    kbs, kv = cache.shape
    if kbs != bs or hq % kv != 0:
        raise ValueError(f"q {tuple(q.shape)} does not match cache (bs={kbs}, kv={kv})")
    n_groups = cache.n_groups if n_groups is None else int(n_groups)
    res_len = cache.res_len if res_len is None else int(res_len)
    sm_scale = 1.0 / math.sqrt(HEAD_DIM) if sm_scale is None else float(sm_scale)
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype must be bfloat16 or float32; got {out_dtype}")
    if out is None:
        out = torch.empty(bs, hq, HEAD_DIM, dtype=out_dtype, device=q.device)
    elif out.dtype != out_dtype or not out.is_contiguous() or out.numel() != bs * hq * HEAD_DIM:
        raise ValueError("out must be a contiguous [bs, hq, 128] tensor of out_dtype")
    lse = torch.empty(bs, hq, dtype=torch.float32, device=q.device) if return_lse else None
    # the residual rows may be a row window of a larger buffer: its row
    # stride per head is the buffer's capacity
    r_cap = cache.k_res.stride(1) // HEAD_DIM
    for name, t in (("k_res", cache.k_res), ("v_res", cache.v_res)):
        if t.stride(3) != 1 or t.stride(2) != HEAD_DIM or t.stride(1) != r_cap * HEAD_DIM or \
                t.stride(0) != kv * r_cap * HEAD_DIM or t.shape[2] < res_len:
            raise ValueError(f"{name} must be a token window of a contiguous [bs, kv, R_cap, 128] buffer holding "
                             f"res_len={res_len} rows")
    ws = workspace
    if ws is None:
        ws = _workspace(q.device, _decode_ws_bytes(bs, hq, kv, n_groups, res_len, n_splits))
    args = (ptr(q3), q3.stride(0), q3.stride(1),
            ptr(cache.groups), cache.g_cap,
            ptr(cache.k_res), ptr(cache.v_res), r_cap,
            bs, hq, kv, n_groups, res_len, sm_scale,
            ptr(out), int(out_dtype == torch.float32), ptr(lse), n_splits,
            ptr(ws), ws.numel() * ws.element_size())
    owners = (q3, cache.groups, cache.k_res, cache.v_res, out, lse, ws)
    if out.dim() != 3 or out.shape[1] != hq:
        out = out.view(bs, hq, HEAD_DIM)
    out = out.unsqueeze(1) if squeeze else out
    return args, ((out, lse) if return_lse else out), owners


def kivi4_sparse_attention(q: torch.Tensor, cache: Kivi4Cache, pages: torch.Tensor,
                           n_groups: int | None = None, res_len: int | None = None,
                           sm_scale: float | None = None, out: torch.Tensor | None = None,
                           out_dtype: torch.dtype | None = None, n_splits: int = 0,
                           workspace: torch.Tensor | None = None, return_lse: bool = False):
    """Decode attention of q (bf16 [bs, hq, 128] or [bs, 1, hq, 128]) over the
    16-token pages listed in ``pages`` (int64 [bs, kv, n_sel]; page P = tokens
    16P .. 16P+15 of the quantized region) plus the bf16 residual window:
    the result of gathering those tokens and attending over them
    (S:1723-1772 after the Quest pick of S:2195-2240).  Sorted page lists let
    both halves of a 32-token group share one tile.  With ``return_lse`` also
    the fp32 natural-log LSE [bs, hq]."""
    args, ret, _ = _sparse_args(q, cache, pages, n_groups, res_len, sm_scale, out, out_dtype, n_splits,
                                workspace, return_lse, copies=True)
    check(lib().zkv_kivi4_sparse_attention(*args, stream_of(q)))
    return ret


class SparseAttentionPlan:
    """``kivi4_sparse_attention`` with its checks done once for fixed buffers
    (a decode loop: new query, page-list and cache contents, the same
    tensors): ``run()`` is one C-ABI call on the current stream and returns
    the output (and LSE).  The page list must have a contiguous last dim (the
    plan reads it in place); the tensors must stay alive and keep their
    shapes and strides; without a ``workspace`` the plan takes the one cached
    for the stream current at creation, so run it on that stream."""

    def __init__(self, q, cache, pages, n_groups=None, res_len=None, sm_scale=None, out=None, out_dtype=None,
                 n_splits=0, workspace=None, return_lse=False):
        self._q = q
        self._args, self.out, self._keep = _sparse_args(q, cache, pages, n_groups, res_len, sm_scale, out,
                                                        out_dtype, n_splits, workspace, return_lse, copies=False)
        self._fn = lib().zkv_kivi4_sparse_attention

    def run(self):
        check(self._fn(*self._args, stream_of(self._q)))
        return self.out


def _sparse_args(q, cache, pages, n_groups, res_len, sm_scale, out, out_dtype, n_splits, workspace, return_lse,
                 copies: bool):
    """Checked arguments of zkv_kivi4_sparse_attention (all but the stream),
    the result to return and the tensors the pointers belong to; with
    ``copies`` False a page list that would need a contiguous copy is an
    error."""
    require_gpu(q, pages)
    _check_bf16("q", q)
    squeeze = q.dim() == 4
    if squeeze and q.shape[1] != 1:
        raise ValueError("decode attention takes one query token per sequence")
    q3 = q[:, 0] if squeeze else q
    _check_last_contig("q", q3)
    bs, hq, _ = q3.shape
    kbs, kv = cache.shape
    if kbs != bs or hq % kv != 0:
        raise ValueError(f"q {tuple(q.shape)} does not match cache (bs={kbs}, kv={kv})")
    if pages.dtype != torch.int64 or pages.dim() != 3 or pages.shape[0] != bs or pages.shape[1] != kv:
        raise ValueError("pages must be int64 [bs, kv, n_sel]")
    if pages.shape[2] > 1 and pages.stride(2) != 1:
        if not copies:
            raise ValueError("a sparse-attention plan reads the page list in place: its last dim must be contiguous")
        pages = pages.contiguous()
    n_sel = pages.shape[2]
    n_groups = cache.n_groups if n_groups is None else int(n_groups)
    res_len = cache.res_len if res_len is None else int(res_len)
    sm_scale = 1.0 / math.sqrt(HEAD_DIM) if sm_scale is None else float(sm_scale)
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype must be bfloat16 or float32; got {out_dtype}")
    if out is None:
        out = torch.empty(bs, hq, HEAD_DIM, dtype=out_dtype, device=q.device)
    elif out.dtype != out_dtype or not out.is_contiguous() or out.numel() != bs * hq * HEAD_DIM:
        raise ValueError("out must be a contiguous [bs, hq, 128] tensor of out_dtype")
    lse = torch.empty(bs, hq, dtype=torch.float32, device=q.device) if return_lse else None
    ws = workspace
    if ws is None:
        ws = _workspace(q.device, _sparse_ws_bytes(bs, hq, kv, n_sel, res_len, n_splits))
    args = (ptr(q3), q3.stride(0), q3.stride(1),
            ptr(cache.groups), cache.g_cap,
            ptr(cache.k_res), ptr(cache.v_res), cache.r_cap,
            bs, hq, kv, n_groups, res_len, ptr(pages), pages.stride(0), pages.stride(1), n_sel, sm_scale,
            ptr(out), int(out_dtype == torch.float32), ptr(lse), n_splits,
            ptr(ws), ws.numel() * ws.element_size())
    owners = (q3, cache.groups, cache.k_res, cache.v_res, pages, out, lse, ws)
    if out.dim() != 3 or out.shape[1] != hq:
        out = out.view(bs, hq, HEAD_DIM)
    out = out.unsqueeze(1) if squeeze else out
    return args, ((out, lse) if return_lse else out), owners


MAX_LIST_TOKENS = 1024   # token-list entries per (b, kv) of kivi4_token_attention


def kivi4_token_attention(q: torch.Tensor, groups: torch.Tensor, n_groups: int, k_rows: torch.Tensor,
                          v_rows: torch.Tensor, toks: torch.Tensor | None, tail_row0: int, n_tail: int,
                          near_row0: int, near_len: int, sm_scale: float | None = None,
                          out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                          n_splits: int = 0, workspace: torch.Tensor | None = None, return_lse: bool = False):
    """Decode attention of q (bf16 [bs, hq, 128] or [bs, 1, hq, 128]) over a
    token list plus contiguous bf16 rows, in one launch: the 4-bit
    counterpart of gathering sink + local + the selected tokens and calling
    flash_attn_with_kvcache (S:1723-1772).

    ``toks`` int64 [bs, kv, n_tok] (n_tok <= 1024, any order): an id in
    [0, 32 n_groups) is that token of the Format Q records ``groups`` (int32
    [bs, kv, G_cap, 1280]); an id in [32 n_groups, 32 n_groups + n_tail) is the
    bf16 row ``tail_row0 + id - 32 n_groups`` of ``k_rows`` / ``v_rows`` (bf16
    [bs, kv, n_rows, 128], rows 16-byte aligned); other ids are skipped; a
    repeated id counts again.  Rows [near_row0, near_row0 + near_len) follow.
    Output has q's shape and ``out_dtype`` (bf16 default, or float32); with
    ``return_lse`` also the fp32 natural-log LSE [bs, hq]."""
    require_gpu(q, groups, k_rows, v_rows, toks)
    _check_bf16("q", q)
    squeeze = q.dim() == 4
    if squeeze and q.shape[1] != 1:
        raise ValueError("decode attention takes one query token per sequence")
    q3 = q[:, 0] if squeeze else q
    _check_last_contig("q", q3)
    bs, hq, _ = q3.shape
    if groups.dtype != torch.int32 or groups.dim() != 4 or groups.shape[-1] != RECORD_WORDS or \
            not groups.is_contiguous():
        raise ValueError("groups must be contiguous int32 [bs, kv, G_cap, 1280]")
    gbs, kv, g_cap, _ = groups.shape
    if gbs != bs or hq % kv != 0:
        raise ValueError(f"q {tuple(q.shape)} does not match the cache (bs={gbs}, kv={kv})")
    if not 0 <= int(n_groups) <= g_cap:
        raise ValueError(f"n_groups {n_groups} outside [0, {g_cap}]")
    for name, t in (("k_rows", k_rows), ("v_rows", v_rows)):
        _check_bf16(name, t)
        if t.dim() != 4 or tuple(t.shape[:2]) != (bs, kv) or t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
            raise ValueError(f"{name} must be bf16 [bs, kv, n_rows, 128] with a contiguous last dim")
        if any(st % 8 for st in t.stride()[:3]) or t.data_ptr() % 16:
            raise ValueError(f"{name} rows must be 16-byte aligned")
    if k_rows.shape != v_rows.shape:
        raise ValueError("k_rows / v_rows shape mismatch")
    n_rows = k_rows.shape[2]
    if toks is None:
        toks = torch.empty(bs, kv, 0, dtype=torch.int64, device=q.device)
    if toks.dtype != torch.int64 or toks.dim() != 3 or tuple(toks.shape[:2]) != (bs, kv):
        raise ValueError("toks must be int64 [bs, kv, n_tok]")
    if toks.shape[2] > MAX_LIST_TOKENS:
        raise ValueError(f"at most {MAX_LIST_TOKENS} listed tokens per (b, kv); got {toks.shape[2]}")
    if toks.shape[2] > 1 and toks.stride(2) != 1:
        toks = toks.contiguous()
    sm_scale = 1.0 / math.sqrt(HEAD_DIM) if sm_scale is None else float(sm_scale)
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype must be bfloat16 or float32; got {out_dtype}")
    if out is None:
        out = torch.empty(bs, hq, HEAD_DIM, dtype=out_dtype, device=q.device)
    elif out.dtype != out_dtype or not out.is_contiguous() or out.numel() != bs * hq * HEAD_DIM:
        raise ValueError("out must be a contiguous [bs, hq, 128] tensor of out_dtype")
    lse = torch.empty(bs, hq, dtype=torch.float32, device=q.device) if return_lse else None
    L = lib()
    n_tok = toks.shape[2]
    need = L.zkv_kivi4_token_attention_workspace_size(bs, hq, kv, n_tok, int(near_len), n_splits)
    ws = _workspace(q.device, need) if workspace is None else workspace
    ks, vs = k_rows.stride(), v_rows.stride()
    check(L.zkv_kivi4_token_attention(
        ptr(q3), q3.stride(0), q3.stride(1), ptr(groups), g_cap, int(n_groups),
        ptr(k_rows), ks[0], ks[1], ks[2], ptr(v_rows), vs[0], vs[1], vs[2], n_rows,
        ptr(toks), toks.stride(0), toks.stride(1), n_tok, int(tail_row0), int(n_tail), int(near_row0),
        int(near_len), bs, hq, kv, sm_scale, ptr(out), int(out_dtype == torch.float32), ptr(lse), n_splits,
        ptr(ws), ws.numel() * ws.element_size(), stream_of(q)))
    out = out.view(bs, hq, HEAD_DIM)
    out = out.unsqueeze(1) if squeeze else out
    return (out, lse) if return_lse else out


def kivi4_attention_partial(q: torch.Tensor, cache: Kivi4Cache, n_groups: int, res_len: int,
                            sm_scale: float | None = None, n_splits: int = 0,
                            workspace: torch.Tensor | None = None):
    """Stage 1 only (per-split partial o / m / l); returns (workspace, n_splits).
    ``attention_merge`` finishes the op.  Used for split-level timing and as the
    building block of a context-sharded decode."""
    import ctypes
    bs, hq, _ = q.shape
    kv = cache.shape[1]
    sm_scale = 1.0 / math.sqrt(HEAD_DIM) if sm_scale is None else float(sm_scale)
    L = lib()
    need = L.zkv_kivi4_attention_workspace_size(bs, hq, kv, n_groups, res_len, n_splits)
    ws = _workspace(q.device, need) if workspace is None else workspace
    used = ctypes.c_int(0)
    check(L.zkv_kivi4_attention_partial(
        ptr(q), q.stride(0), q.stride(1),
        ptr(cache.groups), cache.g_cap,
        ptr(cache.k_res), ptr(cache.v_res), cache.r_cap,
        bs, hq, kv, n_groups, res_len, sm_scale, n_splits,
        ptr(ws), ws.numel() * ws.element_size(), ctypes.addressof(used), stream_of(q)))
    return ws, used.value


def attention_merge(workspace: torch.Tensor, bs: int, hq: int, kv: int, n_splits: int,
                    out: torch.Tensor) -> torch.Tensor:
    """Stage 2: LSE merge of the split partials into ``out`` ([bs, hq, 128] bf16 or fp32)."""
    check(lib().zkv_attention_merge(ptr(workspace), bs, hq, kv, n_splits, ptr(out),
                                    int(out.dtype == torch.float32), stream_of(out)))
    return out


def partial_chunk_kivi_qk_dense_sparse_cuda(chunk_ids, dense_mask, packed_K, chunk_min, chunk_max,
                                            raw_q, dense_topk, sparse_topk, group_size, out_scores,
                                            out_indices, kernel=None, out_width=None) -> None:
    """KIVI stage-2 scorer on a Format R cache, in place (signature of
    Z/cache_hub/kivi/kivi_qk_dot_ops.py:29-67; ``kernel`` is ignored).

    ``out_width`` (an extension, default group_size): slot i's lanes
    0 .. out_width-1 go to ``i * out_width`` of the outputs, which then need
    nk * out_width entries; max(dense_topk, sparse_topk) <= out_width <=
    group_size.  Only the (-1e30, 0) fillers past the kept lanes are left
    out, so a top-k over the outputs that takes no filler is unchanged."""
    require_gpu(chunk_ids, dense_mask, packed_K, chunk_min, chunk_max, raw_q, out_scores, out_indices)
    if chunk_ids.dtype != torch.int64:
        chunk_ids = chunk_ids.to(torch.int64)
    if dense_mask.dtype != torch.bool:
        dense_mask = dense_mask.bool()
    if packed_K.dtype != torch.int32:
        raise TypeError(f"packed_K must be int32; got {packed_K.dtype}")
    for name, t in (("chunk_min", chunk_min), ("chunk_max", chunk_max), ("raw_q", raw_q)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16; got {t.dtype}")
    if out_scores.dtype != torch.float32:
        raise TypeError(f"out_scores must be float32; got {out_scores.dtype}")
    if out_indices.dtype != torch.int64:
        raise TypeError(f"out_indices must be int64; got {out_indices.dtype}")
    g = int(group_size)
    if g not in (8, 16):
        raise ValueError(f"group_size must be 8 or 16; got {group_size}")
    if packed_K.dim() != 5 or packed_K.shape[3] != 16 or packed_K.shape[4] != g:
        raise RuntimeError("packed_K must be chunk-major [bs, kv, n_chunks, 16, group_size]")
    if packed_K.stride(4) != 1 or packed_K.stride(3) != g or packed_K.stride(2) != 16 * g:
        raise RuntimeError("packed_K inner [n_chunks, 16, group_size] must be contiguous")
    if chunk_min.stride() != chunk_max.stride() or chunk_min.stride(3) != 1 or chunk_min.stride(2) != 128:
        raise RuntimeError("chunk_min / chunk_max must share strides with contiguous [.., 128] rows")
    for t in (chunk_ids, dense_mask, raw_q, out_scores, out_indices):
        if t.stride(-1) != 1:
            raise RuntimeError("last dims must be contiguous")
    if out_scores.stride()[:2] != out_indices.stride()[:2]:
        raise RuntimeError("out_scores / out_indices must share batch / head strides")
    bs, kv, nk = chunk_ids.shape
    w = g if out_width is None else int(out_width)
    if out_scores.shape[2] < nk * w or out_indices.shape[2] < nk * w:
        raise RuntimeError(f"outputs too small: need {nk * w}")
    args = (ptr(chunk_ids), chunk_ids.stride(0), chunk_ids.stride(1),
            ptr(dense_mask), dense_mask.stride(0), dense_mask.stride(1),
            ptr(packed_K), packed_K.stride(0), packed_K.stride(1), packed_K.shape[2],
            ptr(chunk_min), ptr(chunk_max), chunk_min.stride(0), chunk_min.stride(1), chunk_min.shape[2],
            ptr(raw_q), raw_q.stride(0), raw_q.stride(1), int(dense_topk), int(sparse_topk), g)
    tail = (ptr(out_scores), ptr(out_indices), out_scores.stride(0), out_scores.stride(1), bs, kv, nk,
            stream_of(raw_q))
    if w == g:
        check(lib().zkv_kivi_qk_dense_sparse(*args, *tail))
    else:
        check(lib().zkv_kivi_qk_dense_sparse_compact(*args, w, *tail))
