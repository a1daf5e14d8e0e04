"""ParisKV-compatible 4-bit RaBitQ codes (1-bit sign + 3-bit magnitude per
dimension), their query blocks and the 4-bit approximate-inner-product rerank
(oracle; TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

Restated from the reference's torch code, one torch op at a time, with each
rounding point kept (bf16 values are float32 arrays on the bf16 grid):

* key encode, PC:1130-1195 (``batch_encode``), PC = Z/cache_hub/polar_cache.py:
  - ``key_norm = vector_norm(Y)`` (PC:1143): fp32 sum of squares (in the
    order of ``_row_norm_bf16``), sqrt, rounded to bf16;
  - ``Y / key_norm.clamp(min=1e-8)`` (PC:1144): fp32 division, bf16;
  - one SRHT round (PC:1148-1151): ``* signs`` (exact for +-1), then
    ``hadamard_transform(scale=1/sqrt(128))``: the fp32 butterfly of
    Z/cache_hub/hadamard_fallback.py:16-26 (pairs (i, i+h) -> (a+b, a-b),
    h = 1, 2, ..., 64), the fp32 scale, one rounding to bf16;
  - blocks of m = 8 (B = 16); sign bit j of block b = (y >= 0), bit-packed
    with weight 2^j (PC:1156-1160), stored [B, seq];
  - block radius r = vector_norm of the 8 bf16 values (PC:1168): fp32, bf16;
  - ``u = y / r.clamp(min=1e-8)`` (PC:1170-1171), bf16; t = bucketize(|u|,
    thresholds) = number of thresholds strictly below |u| (PC:1179);
  - ``alpha = sum(bf16(a[t] * |u|))`` in fp32, clamp(min=1e-6) (PC:1183-1189);
  - ``weight = (r / alpha) * key_norm`` in fp32, rounded to bf16 (PC:1191-1192);
  - 4-bit value v = (sign << 3) | t, two per byte: (v_odd << 4) | v_even
    (PC:1067-1084), stored [B, seq, 4].
* query blocks, PC:1108-1124 (``_encode_query_blocks``): the same norm,
  division and SRHT; q_blocks bf16 [B, 8], q_norm bf16.
* rerank score, Z/cache_hub/rerank/rerank.cu:52-143 (the CUDA kernel the
  production path calls, PC:1768-1779), whose order the reference's own test
  fixes (Z/cache_hub/rerank/test_rerank_topk.py:60-113): the 8 decoded values
  +-centers[t] (bit 3 set: +), each product bf16(value * q) and each running
  sum bf16(sum + product) from 0, per block bf16(dot * weight) added in block
  order, then bf16(res * q_norm).
* top-k: ``torch.topk(approx_scores, final_topk)`` then a gather of the
  candidate indices (PC:1822-1825); the build returns that set in
  increasing candidate position, ties to the earlier position (torch.topk
  leaves the order of ties open).

The magnitude levels are the Lloyd-Max values hard-coded at PC:266-270 (as
bf16); the reference's codebooks/magnitude_levels_m8_4bit.json holds a
slightly different 8-level set that the production path does not use.
"""
from __future__ import annotations

import numpy as np

from .numerics import BF16_1EM8, bf16r, f32

D = 128
M = 8
NB = D // M
MAG_THRESHOLDS = bf16r(np.array([0.0843, 0.1698, 0.2578, 0.3499, 0.4487, 0.5585, 0.6901], dtype=np.float32))
MAG_CENTERS = bf16r(np.array([0.0420, 0.1266, 0.2130, 0.3025, 0.3973, 0.5001, 0.6169, 0.7633], dtype=np.float32))
HADAMARD_SCALE = np.float32(1.0 / np.sqrt(128.0))


def _seq_sum(v: np.ndarray) -> np.ndarray:
    """fp32 sum along the last axis in index order."""
    acc = np.zeros(v.shape[:-1], dtype=np.float32)
    for i in range(v.shape[-1]):
        acc = (acc + v[..., i]).astype(np.float32)
    return acc


def _norm_bf16(x: np.ndarray) -> np.ndarray:
    """vector_norm of 8 bf16 values: fp32 squares summed in index order, sqrt, bf16."""
    return bf16r(np.sqrt(_seq_sum((x * x).astype(np.float32))).astype(np.float32))


def _row_norm_bf16(x: np.ndarray) -> np.ndarray:
    """vector_norm of bf16 rows [..., 128] in the gfx950 kernel's order: each
    8-dimension block summed in index order, then the 16 block sums by a
    butterfly (blocks b and b + 8, then + 4, + 2, + 1); sqrt; bf16.  (The
    reference's fp32 reduction order is torch's; the result is rounded to
    bf16, and the committed reference vectors agree bit for bit.)"""
    s = _seq_sum((x * x).astype(np.float32).reshape(x.shape[:-1] + (NB, M)))
    w = NB
    while w > 1:
        w //= 2
        s = (s[..., :w] + s[..., w:2 * w]).astype(np.float32)
    return bf16r(np.sqrt(s[..., 0]).astype(np.float32))


def fwht_f32(x: np.ndarray) -> np.ndarray:
    """The fp32 butterfly of hadamard_fallback.py:16-23 (no scale)."""
    y = f32(x).copy()
    n = y.shape[-1]
    h = 1
    while h < n:
        y = y.reshape(y.shape[:-1] + (n // (2 * h), 2, h))
        a, b = y[..., 0, :], y[..., 1, :]
        y = np.concatenate([(a + b).astype(np.float32), (a - b).astype(np.float32)], axis=-1)
        y = y.reshape(y.shape[:-2] + (n,))
        h *= 2
    return y


def srht_unit(x: np.ndarray, signs: np.ndarray):
    """bf16 rows [..., 128] -> (bf16 norm [...], bf16 rotated unit rows [..., 128])."""
    x = bf16r(x)
    nrm = _row_norm_bf16(x)
    xn = bf16r((x / np.maximum(nrm, BF16_1EM8)[..., None]).astype(np.float32))
    y = fwht_f32((xn * bf16r(signs)).astype(np.float32))
    return nrm, bf16r((y * HADAMARD_SCALE).astype(np.float32))


def bucketize(absu: np.ndarray) -> np.ndarray:
    """torch.bucketize(v, thresholds), right=False: count of thresholds < v."""
    return (absu[..., None] > MAG_THRESHOLDS).sum(axis=-1).astype(np.uint8)


def encode_keys(keys: np.ndarray, signs: np.ndarray):
    """keys bf16 [N, 128] -> (codebook uint8 [16, N], packed uint8 [16, N, 4],
    weight bf16 [16, N] as float32)."""
    n = keys.shape[0]
    knorm, y = srht_unit(keys, signs)
    yb = y.reshape(n, NB, M)
    bits = (yb >= 0).astype(np.uint8)
    code = (bits << np.arange(M, dtype=np.uint8)).sum(axis=-1).astype(np.uint8)
    r = _norm_bf16(yb)
    u = bf16r((yb / np.maximum(r, BF16_1EM8)[..., None]).astype(np.float32))
    absu = np.abs(u)
    t = bucketize(absu)
    prod = bf16r((MAG_CENTERS[t] * absu).astype(np.float32))
    alpha = np.maximum(_seq_sum(prod), np.float32(1e-6)).astype(np.float32)
    w = bf16r(((r / alpha).astype(np.float32) * knorm[:, None]).astype(np.float32))
    v = (bits << 3) | t
    packed = ((v[..., 1::2] << 4) | v[..., 0::2]).astype(np.uint8)
    return code.T.copy(), packed.transpose(1, 0, 2).copy(), w.T.copy()


def encode_query(q: np.ndarray, signs: np.ndarray):
    """q bf16 [..., 128] -> (q_blocks bf16 [..., 16, 8], q_norm bf16 [...])."""
    qn, y = srht_unit(q, signs)
    return y.reshape(y.shape[:-1] + (NB, M)), qn


def decode_packed(packed: np.ndarray) -> np.ndarray:
    """packed uint8 [..., 4] -> the 8 bf16 values +-centers[t] (rerank.cu:108-124)."""
    v = np.stack([packed & 0x0F, packed >> 4], axis=-1).reshape(packed.shape[:-1] + (M,))
    mag = MAG_CENTERS[v & 7]
    return np.where(v & 8, mag, -mag).astype(np.float32)


def rerank_scores(cand: np.ndarray, packed: np.ndarray, weight: np.ndarray, q_blocks: np.ndarray,
                  q_norm) -> np.ndarray:
    """Scores of candidate keys cand [C] (indices into seq) of one (b, kv):
    packed [16, seq, 4], weight bf16 [16, seq], q_blocks bf16 [16, 8],
    q_norm bf16 -> bf16 [C] (as float32).  An index outside [0, seq) scores
    -inf (the build's rule; the reference reads out of bounds)."""
    ok = (cand >= 0) & (cand < packed.shape[1])
    cand = np.where(ok, cand, 0)
    res = np.zeros(cand.shape[0], dtype=np.float32)
    for b in range(NB):
        vals = decode_packed(packed[b, cand])                 # [C, 8]
        dot = np.zeros(cand.shape[0], dtype=np.float32)
        for j in range(M):
            dot = bf16r((dot + bf16r((vals[:, j] * q_blocks[b, j]).astype(np.float32))).astype(np.float32))
        res = bf16r((res + bf16r((dot * weight[b, cand]).astype(np.float32))).astype(np.float32))
    res = bf16r((res * np.float32(q_norm)).astype(np.float32))
    return np.where(ok, res, np.float32(-np.inf)).astype(np.float32)


def topk_gather(scores: np.ndarray, cand: np.ndarray, k: int) -> np.ndarray:
    """The k largest scores [C] (ties: the earlier position), as candidate
    indices in increasing position order (the set ``torch.topk`` + gather
    picks at PC:1822-1825 up to the order of ties; zkv_topk's order)."""
    order = np.lexsort((np.arange(scores.shape[0]), -scores.astype(np.float64)))[:k]
    return cand[np.sort(order)]
