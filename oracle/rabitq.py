"""RaBitQ 1-bit sign codes, XOR/popcount estimate, top-k and exact rerank (oracle;
TEST INFRASTRUCTURE ONLY, see oracle/__init__.py).

The reference's production RaBitQ path (ParisKV) keeps 4-bit sign+magnitude
codes; the north star asks for the 1-bit variant, which the build defines
from the reference's pieces:

* rotation: one SRHT round, y = H (sigma * x), H the Sylvester Walsh-Hadamard
  matrix applied by the butterfly of Z/cache_hub/hadamard_fallback.py:16-23
  (pairs (i, i+h) -> (a+b, a-b), h = 1, 2, ..., 64), sigma a seeded +-1
  vector (PC:79-93 seeds its signs; the 1/sqrt(D) scale of PC:1150 is dropped:
  only signs and ratios are used);
* code: bit b of byte j is (y[8j+b] >= 0) (PC:1156-1160), 16 bytes per key;
* factors (fp16): norm = ||x||, corr = ||y|| sqrt(D) / sum|y| = 1 / <o_bar, o>
  (o = y/||y||, o_bar = sign(y)/sqrt(D));
* estimate: <q, k> ~ nk*ck * nq*cq * (D - 2 popc(xq ^ xk)) / D, the sign-sign
  inner product identity of Z/cache_hub/rerank/coarse_2bit_score.cu:12-16
  (sum_d s_q s_k = D - 2 N(q_s ^ k_s)) with both RaBitQ corrections;
* exact rerank: fp32 dot of the fp16 query and key.

Every fp32 reduction below fixes its order (it is the gfx950 kernel's).
"""
from __future__ import annotations

import numpy as np

from .numerics import f16_bits, f16_to_f32, f32

D = 128


def srht_signs(seed: int = 42, d: int = D) -> np.ndarray:
    """Seeded +-1 vector (float32)."""
    return np.where(np.random.default_rng(seed).integers(0, 2, size=d) == 1, 1.0, -1.0).astype(np.float32)


def fwht(x: np.ndarray) -> np.ndarray:
    """Unnormalised Walsh-Hadamard transform along the last axis, float32."""
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


def _seq_sum(v: np.ndarray) -> np.ndarray:
    acc = np.zeros(v.shape[:-1], dtype=np.float32)
    for i in range(v.shape[-1]):
        acc = (acc + v[..., i]).astype(np.float32)
    return acc


def encode(x_f16: np.ndarray, signs: np.ndarray):
    """x [N, 128] fp16 bit patterns (uint16) -> (codes uint8 [N, 16],
    factors uint16 fp16 bits [N, 2] = (norm, corr))."""
    x = f16_to_f32(x_f16)
    y = fwht((x * signs).astype(np.float32))
    bits = (y >= 0).astype(np.uint8).reshape(-1, 16, 8)
    codes = (bits << np.arange(8, dtype=np.uint8)).sum(axis=-1).astype(np.uint8)
    norm = np.sqrt(_seq_sum((x * x).astype(np.float32))).astype(np.float32)
    ysq = _seq_sum((y * y).astype(np.float32))
    yabs = _seq_sum(np.abs(y))
    corr = (np.sqrt(ysq).astype(np.float32) * np.float32(np.sqrt(np.float32(D)))).astype(np.float32)
    corr = np.where(yabs > 0, (corr / np.where(yabs > 0, yabs, 1)).astype(np.float32), np.float32(0))
    fac = np.stack([f16_bits(norm), f16_bits(corr.astype(np.float32))], axis=-1)
    return codes, fac


_POPC8 = np.array([bin(i).count("1") for i in range(256)], dtype=np.int32)


def popcount_distance(codes_q: np.ndarray, codes_k: np.ndarray) -> np.ndarray:
    """popc(xq ^ xk) for every (query, key): [Q, N] int32 (byte table lookup)."""
    out = np.zeros((codes_q.shape[0], codes_k.shape[0]), dtype=np.int32)
    for j in range(codes_q.shape[1]):
        out += _POPC8[np.bitwise_xor(codes_q[:, None, j], codes_k[None, :, j])]
    return out


def estimate(codes_q, fac_q, codes_k, fac_k) -> np.ndarray:
    """est[q, k] = ((nk*ck) * (nq*cq)) * (D - 2 popc) * 2^-7, each product a
    float32 op in that order."""
    p = popcount_distance(codes_q, codes_k)
    fk = (f16_to_f32(fac_k[:, 0]) * f16_to_f32(fac_k[:, 1])).astype(np.float32)
    fq = (f16_to_f32(fac_q[:, 0]) * f16_to_f32(fac_q[:, 1])).astype(np.float32)
    t = (fq[:, None] * fk[None, :]).astype(np.float32)
    t = (t * (D - 2 * p).astype(np.float32)).astype(np.float32)
    return (t * np.float32(2.0 ** -7)).astype(np.float32)


def exact_scores(q_f16: np.ndarray, k_f16: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """Exact dot of query i with keys idx[i] (fp16 inputs, exact fp32
    products): 16 lanes sum 8 dims each left to right, then a xor butterfly
    8, 4, 2, 1.  q [Q, 128], k [N, 128] fp16 bits, idx [Q, C] -> [Q, C]."""
    q = f16_to_f32(q_f16)
    k = f16_to_f32(k_f16)[idx]                                   # [Q, C, 128]
    prod = (q[:, None, :] * k).astype(np.float32).reshape(idx.shape + (16, 8))
    s = prod[..., 0]
    for i in range(1, 8):
        s = (s + prod[..., i]).astype(np.float32)
    for off in (8, 4, 2, 1):
        s = (s[..., :off] + s[..., off:2 * off]).astype(np.float32)
    return s[..., 0]


def search(q_f16, k_f16, codes_k, fac_k, signs, topk: int):
    """Full pipeline: encode queries, estimate, top-k by estimate (ties by
    lower index), exact rerank, order by (exact desc, index asc).
    Returns (cand_idx [Q, topk] increasing, final_idx [Q, topk], final_scores)."""
    from .select import topk_indices
    codes_q, fac_q = encode(q_f16, signs)
    est = estimate(codes_q, fac_q, codes_k, fac_k)
    cand = topk_indices(est, topk)
    ex = exact_scores(q_f16, k_f16, cand)
    order = np.lexsort((cand, -ex.astype(np.float64)), axis=-1)
    final_idx = np.take_along_axis(cand, order, axis=-1)
    final_sc = np.take_along_axis(ex, order, axis=-1)
    return cand, final_idx, final_sc


def clustered_unit_keys(rng, n: int, n_clusters: int = 64, sigma: float = 0.1, d: int = D):
    """Seeded unit-norm cluster data, fp16 bit patterns."""
    centres = rng.standard_normal((n_clusters, d)).astype(np.float32)
    centres /= np.linalg.norm(centres, axis=1, keepdims=True)
    lab = rng.integers(0, n_clusters, size=n)
    x = centres[lab] + np.float32(sigma) * rng.standard_normal((n, d)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    return f16_bits(x)
