"""RaBitQ 1-bit sign codes, estimate, top-k and exact rerank on gfx950.

The reference's RaBitQ path (ParisKV) stores 4-bit sign + magnitude codes per
8-dim block (``PC:1130-1195``) and reranks candidates with
``rerank_rabitq_ref`` (``Z/cache_hub/rerank/rerank.py:205-274``: coarse filter ->
approximate score -> top-k).  This module keeps one sign bit per rotated
dimension (16 bytes per 128-dim key) with fp16 (norm, correction) factors:

* ``rabitq_encode``: SRHT (one +-1 sign round, then the Walsh-Hadamard
  butterfly of ``Z/cache_hub/hadamard_fallback.py:16-23``) and bit-pack of
  ``y >= 0`` as in ``PC:1147-1160``;
* ``rabitq_estimate``: ``((nk*ck) * (nq*cq)) * (128 - 2 popc(xq ^ xk)) / 128``;
* ``rabitq_search``: top-k by estimate (ties to the lower index), exact fp32
  rerank of the fp16 keys, output ordered by (score desc, index asc).

Pools are independent key sets (e.g. one per (batch, kv head)); queries of a
pool are searched against that pool only.
"""
from __future__ import annotations

import torch

from ._lib import check, device_stream, lib, ptr, require_gpu, stream_of

HEAD_DIM = 128
CODE_BYTES = 16


def srht_signs(seed: int = 42, device="cuda") -> torch.Tensor:
    """Seeded +-1 SRHT diagonal (fp32 [128]); the reference draws its signs
    from a seeded torch RNG the same way (``PC:79-93``)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    s = torch.randint(0, 2, (HEAD_DIM,), generator=g).to(torch.float32) * 2 - 1
    return s.to(device)


def _check_signs(signs: torch.Tensor):
    assert signs.dtype == torch.float32 and signs.shape == (HEAD_DIM,) and signs.is_contiguous(), \
        "signs must be a contiguous fp32 [128] tensor"


def rabitq_encode(x: torch.Tensor, signs: torch.Tensor, codes: torch.Tensor | None = None,
                  factors: torch.Tensor | None = None):
    """x fp16 [..., 128] -> (codes uint8 [..., 16], factors fp16 [..., 2] = (norm, corr))."""
    require_gpu(x, signs)
    _check_signs(signs)
    assert x.dtype == torch.float16 and x.shape[-1] == HEAD_DIM, "x must be fp16 [..., 128]"
    lead = x.shape[:-1]
    rows = x.reshape(-1, HEAD_DIM)
    if rows.stride(-1) != 1 or (rows.stride(0) % 8) or (rows.data_ptr() % 16):
        rows = rows.contiguous()
    n = rows.shape[0]
    if codes is None:
        codes = torch.empty(*lead, CODE_BYTES, dtype=torch.uint8, device=x.device)
    if factors is None:
        factors = torch.empty(*lead, 2, dtype=torch.float16, device=x.device)
    assert codes.is_contiguous() and codes.dtype == torch.uint8 and codes.numel() == n * CODE_BYTES
    assert factors.is_contiguous() and factors.dtype == torch.float16 and factors.numel() == n * 2
    check(lib().zkv_rabitq_encode(ptr(rows), rows.stride(0) if n else HEAD_DIM, n, ptr(signs),
                                  ptr(codes), ptr(factors), stream_of(x)))
    return codes, factors


def _pools(t: torch.Tensor, last: int) -> torch.Tensor:
    """[N, last] -> [1, N, last]; [P, N, last] as is."""
    assert t.dim() in (2, 3) and t.shape[-1] == last, f"expected [..., {last}], got {tuple(t.shape)}"
    return t.unsqueeze(0) if t.dim() == 2 else t


def rabitq_estimate(codes_q: torch.Tensor, factors_q: torch.Tensor, codes_k: torch.Tensor,
                    factors_k: torch.Tensor) -> torch.Tensor:
    """Estimate matrix fp32 [P, Q, N] (or [Q, N] for 2-D inputs)."""
    require_gpu(codes_q, factors_q, codes_k, factors_k)
    squeeze = codes_q.dim() == 2
    cq, fq = _pools(codes_q, CODE_BYTES).contiguous(), _pools(factors_q, 2).contiguous()
    ck, fk = _pools(codes_k, CODE_BYTES).contiguous(), _pools(factors_k, 2).contiguous()
    P, Q, _ = cq.shape
    assert ck.shape[0] == P and fq.shape[:2] == cq.shape[:2] and fk.shape[:2] == ck.shape[:2]
    N = ck.shape[1]
    out = torch.empty(P, Q, N, dtype=torch.float32, device=cq.device)
    check(lib().zkv_rabitq_estimate(ptr(cq), ptr(fq), ptr(ck), ptr(fk), P, Q, N, ptr(out),
                                    stream_of(cq)))
    return out[0] if squeeze else out


_WS: dict = {}


def search_workspace(pools: int, queries: int, n: int, topk: int, device) -> torch.Tensor:
    """The search workspace cached per (device, current stream): searches on
    one stream run in order; searches on two streams get two workspaces."""
    nbytes = lib().zkv_rabitq_search_workspace_size(pools, queries, n, topk)
    dev = torch.device(device)
    key = (dev, device_stream(dev))
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        _WS[key] = ws
    return ws


_F16, _U8, _I64, _F32 = torch.float16, torch.uint8, torch.int64, torch.float32


def rabitq_search(q: torch.Tensor, keys: torch.Tensor, codes: torch.Tensor, factors: torch.Tensor,
                  signs: torch.Tensor, topk: int, workspace: torch.Tensor | None = None,
                  out: tuple | None = None):
    """Top-``topk`` keys per query by RaBitQ estimate, reranked exactly.

    q fp16 [P, Q, 128] (or [Q, 128]); keys fp16 [P, N, 128] (or [N, 128]; row
    views with a 16-byte aligned stride are used in place); codes uint8
    [P, N, 16]; factors fp16 [P, N, 2].  Returns (cand_idx int64 [P, Q, topk]
    in increasing index order, final_idx int64 [P, Q, topk], final_scores
    fp32 [P, Q, topk]) with the final pair ordered by (score desc, index asc).
    ``out``: the three output tensors, preallocated with those shapes and
    dtypes (contiguous), written in place and returned.
    """
    args, outs, _ = _search_args(q, keys, codes, factors, signs, topk, workspace, out, copies=True)
    check(lib().zkv_rabitq_search(*args, stream_of(q)))
    return outs


class SearchPlan:
    """``rabitq_search`` with its argument checks done once, for searches
    repeated over the same buffers (a serving loop: new query and key
    contents, the same tensors).  ``run()`` searches the buffers' current
    contents with one C-ABI call on the current stream, allocates nothing and
    returns the output tensors.  q, codes and factors must be contiguous and
    the key rows 16-byte aligned (the plan reads them in place, never a
    copy); the tensors and the workspace must stay alive and keep their
    shapes and strides while the plan is used.  Without a ``workspace`` the
    plan takes the one cached for the stream current at its creation: run it
    on that stream (overlapping searches on one workspace race)."""

    def __init__(self, q, keys, codes, factors, signs, topk, workspace=None, out=None):
        self._q = q
        self._args, self.out, self._keep = _search_args(q, keys, codes, factors, signs, topk, workspace, out,
                                                        copies=False)
        self._fn = lib().zkv_rabitq_search

    def run(self):
        check(self._fn(*self._args, stream_of(self._q)))
        return self.out


def _search_args(q, keys, codes, factors, signs, topk, workspace, out, copies: bool):
    """The checked arguments of zkv_rabitq_search (all but the stream), the
    outputs to return, and the tensors the pointers belong to.  With
    ``copies`` False an operand that would need a contiguous copy is an
    error."""
    # (the checks are ordered so that the common call -- 3-D pools,
    # contiguous operands, preallocated outputs -- costs a few microseconds
    # of host time: the search itself takes ~30 us of device time)
    require_gpu(q, keys, codes, factors, signs)
    _check_signs(signs)
    squeeze = q.dim() == 2
    qq, kk = _pools(q, HEAD_DIM), _pools(keys, HEAD_DIM)
    cc, ff = _pools(codes, CODE_BYTES), _pools(factors, 2)
    if not copies:
        assert qq.is_contiguous() and cc.is_contiguous() and ff.is_contiguous(), \
            "a search plan reads q, codes and factors in place: they must be contiguous"
    qq, cc, ff = qq.contiguous(), cc.contiguous(), ff.contiguous()
    assert qq.dtype == _F16 and kk.dtype == _F16, "q and keys must be fp16"
    assert cc.dtype == _U8 and ff.dtype == _F16
    P, Q, _ = qq.shape
    N = kk.shape[1]
    assert kk.shape[0] == P and cc.shape[0] == P and cc.shape[1] == N and ff.shape[0] == P and \
        ff.shape[1] == N, "pool/key shape mismatch"
    ks0, ks1 = kk.stride(0), kk.stride(1)
    if kk.stride(2) != 1 or ks1 % 8 or ks0 % 8 or kk.data_ptr() % 16:
        assert copies, "a search plan reads the keys in place: their rows must be 16-byte aligned"
        kk = kk.contiguous()
        ks0, ks1 = kk.stride(0), kk.stride(1)
    assert 0 < topk <= N, f"topk={topk} must be in [1, {N}]"
    ws = workspace if workspace is not None else search_workspace(P, Q, N, topk, q.device)
    if out is None:
        cand = torch.empty(P, Q, topk, dtype=_I64, device=q.device)
        fidx = torch.empty_like(cand)
        fsc = torch.empty(P, Q, topk, dtype=_F32, device=q.device)
    else:
        cand, fidx, fsc = out
        shape = (P, Q, topk)
        dev = q.device
        for t, dt in ((cand, _I64), (fidx, _I64), (fsc, _F32)):
            assert t.dtype == dt and t.is_contiguous() and t.numel() == P * Q * topk and t.device == dev, \
                "out tensors: contiguous int64, int64, fp32 with P * Q * topk elements on q's device"
        if cand.shape != shape:
            cand = cand.view(shape)
        if fidx.shape != shape:
            fidx = fidx.view(shape)
        if fsc.shape != shape:
            fsc = fsc.view(shape)
    args = (qq.data_ptr(), kk.data_ptr(), ks0, ks1, cc.data_ptr(), ff.data_ptr(), signs.data_ptr(), P, Q, N,
            topk, cand.data_ptr(), fidx.data_ptr(), fsc.data_ptr(), ws.data_ptr(), ws.numel())
    outs = (cand[0], fidx[0], fsc[0]) if squeeze else (cand, fidx, fsc)
    # the tensors whose pointers the arguments hold (contiguous copies included)
    return args, outs, (qq, kk, cc, ff, signs, ws, cand, fidx, fsc)
