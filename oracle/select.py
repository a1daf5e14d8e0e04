"""Quest page scoring, top-k selection, CDS density / mask and the KIVI stage-2
scorer (oracle; TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

Canonical arithmetic orders (bit-exact targets for the gfx950 kernels):

* quest_chunk_score: lane t of a 32-lane group sums the fp32 products of
  dims 4t..4t+3 left to right, then a xor butterfly 16, 8, 4, 2, 1
  (Z/cache_hub/quest/quest_chunk_score.cu:54-99).  bf16 x bf16 (or bf16 x fp16)
  products are exact in fp32, so this order fixes every bit.
* chunk_density_scores: thread t of 128 holds centroid[t]*q[t]; then
  buf[t] += buf[t + s] for s = 64, 32, ..., 1 (Z/cache_hub/rerank/rerank_topk.cu:599-615).
* kivi_qk_dense_sparse: per token k = bf16(bf16(code*scale) + mn),
  p = bf16(k*q), acc += p in fp32 for d = 0..127 (Z/cache_hub/kivi/kivi_qk_dot.cu:236-284),
  scale = bf16(bf16(mx - mn) / 15) (:193-223), then the 16/8-lane bitonic
  network of :286-303 and the keep / fill rule of :305-319.
* top-k: the reference's radix select (Z/cache_hub/topk/float_topk.cu:51-271)
  returns the top-k *set* in arbitrary order with arbitrary tie choice; the
  build's kernels pick ties by lowest index and return indices in increasing
  index order, which is one valid output of the reference.
"""
from __future__ import annotations

import numpy as np

from .numerics import bf16r, f32

NEG_FILL = np.float32(-1e30)      # kivi_qk_dot.cu:316, rerank_topk.cu:622


# ---------------------------------------------------------------------------
# Quest
# ---------------------------------------------------------------------------
def quest_chunk_score(q: np.ndarray, cmin: np.ndarray, cmax: np.ndarray, n_chunks: int,
                      valid: np.ndarray | None = None) -> np.ndarray:
    """score[b, h, c] = sum_d max(q_d * mn_d, q_d * mx_d) (quest_chunk_score.cu:31-103).

    q [bs, kv, 128]; cmin/cmax [bs, kv, n_max, 128] (bf16 or fp16 values);
    valid [bs, kv, n_max] bool or None.  Returns fp32 [bs, kv, n_chunks].
    """
    qq = f32(q)[:, :, None, :]
    mn = f32(cmin[:, :, :n_chunks])
    mx = f32(cmax[:, :, :n_chunks])
    m = np.maximum(qq * mn, qq * mx).astype(np.float32)          # exact products
    lanes = m.reshape(m.shape[:-1] + (32, 4))
    s = lanes[..., 0]
    for i in range(1, 4):
        s = (s + lanes[..., i]).astype(np.float32)
    for off in (16, 8, 4, 2, 1):
        s = (s[..., :off] + s[..., off:2 * off]).astype(np.float32)
    out = s[..., 0]
    if valid is not None:
        out = np.where(valid[:, :, :n_chunks], out, np.float32(-np.inf)).astype(np.float32)
    return out


def quest_upper_bound_holds(q, keys_chunked, score) -> bool:
    """Invariant: score(c) >= max_{t in c} q . k_t (brute force, float64)."""
    exact = np.einsum("bhd,bhctd->bhct", q.astype(np.float64), keys_chunked.astype(np.float64)).max(-1)
    return bool(np.all(score.astype(np.float64) >= exact - 1e-4 * (1 + np.abs(exact))))


def f16_directed(x: np.ndarray, up: bool) -> np.ndarray:
    """float32 -> fp16 bits rounded toward +inf (up) or -inf."""
    x = f32(x)
    with np.errstate(over="ignore"):
        h = x.astype(np.float16)
    hf = h.astype(np.float32)
    bits = h.view(np.uint16).copy()
    fix = (hf < x) if up else (hf > x)
    fix &= ~np.isnan(x)
    neg = (bits & 0x8000) != 0
    zero = (bits & 0x7FFF) == 0
    step_dn = np.where(neg == up, bits - 1, bits + 1).astype(np.uint16)   # away/toward zero per sign
    step = np.where(zero, np.uint16(0x0001) if up else np.uint16(0x8001), step_dn).astype(np.uint16)
    return np.where(fix, step, bits).astype(np.uint16)


def page_minmax_f16(keys: np.ndarray, page: int = 16):
    """Per-page per-channel min (rounded down) / max (rounded up) as fp16 bits.
    keys [bs, kv, n_tok, 128] (bf16 values) -> [bs, kv, n_tok // page, 128] x2."""
    bs, kv, n, d = keys.shape
    n_pages = n // page
    kp = f32(keys[:, :, :n_pages * page]).reshape(bs, kv, n_pages, page, d)
    return f16_directed(kp.min(axis=3), False), f16_directed(kp.max(axis=3), True)


# ---------------------------------------------------------------------------
# Top-k
# ---------------------------------------------------------------------------
def ordered_key(x: np.ndarray) -> np.ndarray:
    """float32 -> order-preserving uint32 (float_topk.cu:24-27)."""
    u = f32(x).view(np.uint32)
    return np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def topk_indices(scores: np.ndarray, k: int) -> np.ndarray:
    """Top-k along the last axis: largest keys, ties by lowest index, returned
    in increasing index order.  If L <= k: 0..L-1 then -1 (float_topk.cu:35-40)."""
    L = scores.shape[-1]
    flat = scores.reshape(-1, L)
    out = np.full((flat.shape[0], k), -1, dtype=np.int64)
    if L <= k:
        out[:, :L] = np.arange(L)
        return out.reshape(scores.shape[:-1] + (k,))
    keys = ordered_key(flat).astype(np.int64)
    idx = np.arange(L)
    for r in range(flat.shape[0]):
        order = np.lexsort((idx, -keys[r]))          # key desc, index asc
        out[r] = np.sort(order[:k])
    return out.reshape(scores.shape[:-1] + (k,))


def topk_gather_concat(scores, lut, skipped, k: int, out_width: int) -> np.ndarray:
    """out[:k] = lut[topk(scores)], out[k:k+sk] = skipped, 0 sentinel
    (float_topk_gather_concat.cu:65-114)."""
    sel = topk_indices(scores, k)
    g = np.where(sel >= 0, np.take_along_axis(lut, np.maximum(sel, 0), axis=-1), 0)
    out = np.zeros(scores.shape[:-1] + (out_width,), dtype=np.int64)
    out[..., :k] = g
    sk = skipped.shape[-1]
    out[..., k:k + sk] = skipped
    return out


# ---------------------------------------------------------------------------
# CDS density and dense mask
# ---------------------------------------------------------------------------
def chunk_density_scores(chunk_ids: np.ndarray, centroids: np.ndarray, raw_q: np.ndarray) -> np.ndarray:
    """centroid[chunk_id] . q with the 128-thread tree order (rerank_topk.cu:560-624)."""
    n_chunks = centroids.shape[2]
    ids = chunk_ids.astype(np.int64)
    ok = (ids >= 0) & (ids < n_chunks)
    cent = np.take_along_axis(centroids, np.clip(ids, 0, n_chunks - 1)[..., None], axis=2)
    v = (f32(cent) * f32(raw_q)[:, :, None, :]).astype(np.float32)
    s = 64
    while s >= 1:
        v = (v[..., :s] + v[..., s:2 * s]).astype(np.float32)
        s //= 2
    return np.where(ok, v[..., 0], NEG_FILL).astype(np.float32)


def dense_mask_from_topk(positions: np.ndarray, nk: int) -> np.ndarray:
    """mask.fill_(False); mask.scatter_(2, positions, True), out-of-range skipped
    (rerank_topk.cu:926-954)."""
    bs, kv, _ = positions.shape
    m = np.zeros((bs, kv, nk), dtype=bool)
    for b in range(bs):
        for h in range(kv):
            p = positions[b, h]
            m[b, h, p[(p >= 0) & (p < nk)]] = True
    return m


# ---------------------------------------------------------------------------
# KIVI stage-2 scorer
# ---------------------------------------------------------------------------
def bitonic_desc(scores: np.ndarray, idx: np.ndarray):
    """The CHUNK-lane descending bitonic network of kivi_qk_dot.cu:286-303,
    applied along the last axis (length = chunk size)."""
    s = scores.copy()
    t = idx.copy()
    n = s.shape[-1]
    lane = np.arange(n)
    k = 2
    while k <= n:
        j = k // 2
        while j >= 1:
            partner = lane ^ j
            os_, ot = s[..., partner], t[..., partner]
            desc = (lane & k) == 0
            lower = (lane & j) == 0
            want_larger = desc == lower
            swap = np.where(want_larger, os_ > s, os_ < s)
            s = np.where(swap, os_, s)
            t = np.where(swap, ot, t)
            j //= 2
        k *= 2
    return s, t


def kivi_qk_dense_sparse(chunk_ids, dense_mask, packed_K, chunk_min, chunk_max, raw_q,
                         dense_topk: int, sparse_topk: int, group_size: int):
    """partial_chunk_kivi_qk_dense_sparse (kivi_qk_dot.cu:108-320).

    packed_K [bs, kv, n_packed, 16, g] int32 (Format R); returns
    (scores fp32 [bs, kv, nk*g], indices int64 [bs, kv, nk*g]).
    """
    from .kivi import unpack_last_dim
    bs, kv, nk = chunk_ids.shape
    g = group_size
    n_packed = packed_K.shape[2]
    ids = chunk_ids.astype(np.int64)
    in_range = (ids >= 0) & (ids < n_packed)
    cid = np.clip(ids, 0, n_packed - 1)
    pk = np.take_along_axis(packed_K, cid[..., None, None], axis=2)          # [bs, kv, nk, 16, g]
    codes = unpack_last_dim(np.swapaxes(pk, -1, -2)).astype(np.float32)      # [bs, kv, nk, g, 128]
    n_max = chunk_min.shape[2]
    mid = np.clip(ids, 0, n_max - 1)
    mn = np.take_along_axis(f32(chunk_min), mid[..., None], axis=2)[..., None, :]
    mx = np.take_along_axis(f32(chunk_max), mid[..., None], axis=2)[..., None, :]
    scale = bf16r(bf16r(mx - mn) / np.float32(15.0))
    k = bf16r(bf16r(codes * scale) + mn)
    p = bf16r(k * f32(raw_q)[:, :, None, None, :])
    acc = np.zeros(p.shape[:-1], dtype=np.float32)
    for d in range(p.shape[-1]):
        acc = (acc + p[..., d]).astype(np.float32)
    acc = np.where(in_range[..., None], acc, NEG_FILL).astype(np.float32)
    tok = (ids.astype(np.int32)[..., None] * g + np.arange(g, dtype=np.int32)).astype(np.int64)
    s_sorted, t_sorted = bitonic_desc(acc, tok)
    keep = np.arange(g)[None, None, None, :] < np.where(dense_mask, dense_topk, sparse_topk)[..., None]
    s_out = np.where(keep, s_sorted, NEG_FILL).astype(np.float32)
    t_out = np.where(keep, t_sorted, 0).astype(np.int64)
    return s_out.reshape(bs, kv, nk * g), t_out.reshape(bs, kv, nk * g)


def gqa_mean_query(q: np.ndarray, kv: int) -> np.ndarray:
    """raw_q = bf16(mean over the GQA group) (S:1621-1626): fp32 sum in head
    order, times 1/group (exact for power-of-two groups), RNE to bf16.
    q [bs, hq, 128] -> [bs, kv, 128]."""
    bs, hq, d = q.shape
    grp = hq // kv
    qq = f32(q).reshape(bs, kv, grp, d)
    acc = qq[:, :, 0]
    for i in range(1, grp):
        acc = (acc + qq[:, :, i]).astype(np.float32)
    return bf16r(acc / np.float32(grp))
