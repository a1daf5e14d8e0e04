"""PyTorch-CPU restatements of the C2 decode step, the C3 Quest + sparse
attention step and the C4 RaBitQ search: the CPU baselines of ``bench.py``
(its ``cpu_baseline`` legs).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference's decode path on a CPU, written with torch CPU ops from the
cited formulas (the reference's own files never run here):

  * 4-bit unpack of int32 words, 8 channels per word, channel j of a word in
    bits 4j..4j+3 (quant_pack.py:166-174), and dequant code * scale + zero
    (quant_pack.py:176-198): K per channel over groups of 32 tokens, V per
    token over groups of 32 channels, fp16 scale / zero widened to fp32;
  * the bf16 residual window appended (S:1723-1747 concatenates the cached
    rows before the attention call);
  * fp32 ``scaled_dot_product_attention`` with grouped query heads, standing
    in for flash-attn's math at S:1742-1747 (causal off).

``prepare_c2`` turns a Format Q cache into the reference-style packed words
(untimed: the reference stores its codes token-major); ``decode_attention``
is the timed step.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import kivi as okivi
from .numerics import f16_to_f32


def prepare_c2(k_codes: np.ndarray, k_meta: np.ndarray, v_codes: np.ndarray, v_meta: np.ndarray,
               k_res: np.ndarray, v_res: np.ndarray) -> dict:
    """Format Q arrays ([B, KV, G, ...] as in ``oracle.kivi.Kivi4Cache``) plus
    the bf16 residual (float32 [B, KV, R, 128]) -> torch CPU tensors:
    K words int32 [B, KV, G, 32, 16] (token-major, 8 channels per word),
    V words int32 [B, KV, T, 16], K scale / zero fp32 [B, KV, G, 1, 128],
    V scale / zero fp32 [B, KV, T, 4, 1]."""
    B, KV, G = k_codes.shape[:3]
    kw = np.swapaxes(okivi.k_words_from_lane_order(k_codes), -1, -2)          # [B, KV, G, 32 t, 16 p]
    vc = okivi.v_words_to_codes(v_codes).reshape(B, KV, G * 32, 128)
    vw = okivi.pack_last_dim(vc)                                               # [B, KV, T, 16]
    km = f16_to_f32(k_meta)                                                    # [B, KV, G, 16, 2, 8]
    chan = (np.arange(16)[:, None] * 8 + okivi.KSLOT[None, :]).reshape(-1)
    ks = np.empty((B, KV, G, 128), np.float32)
    kz = np.empty((B, KV, G, 128), np.float32)
    ks[..., chan] = km[..., 0, :].reshape(B, KV, G, 128)
    kz[..., chan] = km[..., 1, :].reshape(B, KV, G, 128)
    vm = f16_to_f32(v_meta)                                                    # [B, KV, G, m, gd, r, 2, i]
    vs = np.moveaxis(vm[..., 0, :], -3, -1).reshape(B, KV, G * 32, 4)
    vz = np.moveaxis(vm[..., 1, :], -3, -1).reshape(B, KV, G * 32, 4)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    return {"kw": t(kw), "vw": t(vw), "ks": t(ks[:, :, :, None, :]), "kz": t(kz[:, :, :, None, :]),
            "vs": t(vs[..., None]), "vz": t(vz[..., None]), "k_res": t(k_res.astype(np.float32)),
            "v_res": t(v_res.astype(np.float32))}


def _unpack(words: torch.Tensor) -> torch.Tensor:
    """int32 words [..., W] -> codes float32 [..., 8 W] (channel 8w + j = bits 4j..4j+3)."""
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    return ((words.unsqueeze(-1) >> shifts) & 15).flatten(-2).to(torch.float32)


def decode_attention(q: torch.Tensor, prep: dict, sm_scale: float, rows=None) -> torch.Tensor:
    """q float32 [B, HQ, 128] -> attention output float32 [len(rows), HQ, 128]
    over the dequantized cache and the residual window, one sequence at a
    time (rows: the batch rows to compute, default all)."""
    B, KV, G = prep["kw"].shape[:3]
    outs = []
    for b in (range(B) if rows is None else rows):
        k = (_unpack(prep["kw"][b]) * prep["ks"][b] + prep["kz"][b]).reshape(KV, G * 32, 128)
        v = (_unpack(prep["vw"][b]).unflatten(-1, (4, 32)) * prep["vs"][b] + prep["vz"][b]).flatten(-2)
        k = torch.cat([k, prep["k_res"][b]], dim=1)
        v = torch.cat([v, prep["v_res"][b]], dim=1)
        o = torch.nn.functional.scaled_dot_product_attention(q[b].unsqueeze(1), k, v, scale=sm_scale,
                                                             enable_gqa=True)
        outs.append(o.squeeze(1))
    return torch.stack(outs)


# ---- C3: Quest bounds -> top-k pages -> attention over the selected pages ----
#
#   * Quest upper bound per page: sum_d max(q_d * min_d, q_d * max_d) over the
#     GQA-mean query (QuestPytorch.quest_chunk_score, quest_ops.py:22-31, with
#     the mean of S:1621-1626), fp16 page metadata widened to fp32;
#   * torch.topk of the page scores (float_topk_3d's role, S:1690-1700),
#     pages in increasing order;
#   * the selected pages' 16 tokens unpacked and dequantized as in C2, then
#     fp32 SDPA with grouped heads (S:1723-1747 over the gathered rows).

def prepare_c3(raw_q: np.ndarray, page_min: np.ndarray, page_max: np.ndarray, k_codes: np.ndarray,
               k_meta: np.ndarray, v_codes: np.ndarray, v_meta: np.ndarray) -> dict:
    """raw_q float32 [B, KV, 128]; page_min / page_max fp16 bits [B, KV, P, 128];
    Format Q arrays as prepare_c2 (no residual window)."""
    B, KV = k_codes.shape[:2]
    z = np.zeros((B, KV, 0, 128), np.float32)
    prep = prepare_c2(k_codes, k_meta, v_codes, v_meta, z, z)
    prep["raw_q"] = torch.from_numpy(np.ascontiguousarray(raw_q, dtype=np.float32))
    prep["pmin"] = torch.from_numpy(f16_to_f32(page_min))
    prep["pmax"] = torch.from_numpy(f16_to_f32(page_max))
    return prep


def quest_scores(prep: dict) -> torch.Tensor:
    """Page upper bounds float32 [B, KV, P]."""
    qv = prep["raw_q"].unsqueeze(2)
    return torch.maximum(qv * prep["pmin"], qv * prep["pmax"]).sum(-1)


def sparse_attention(q: torch.Tensor, prep: dict, pages: torch.Tensor, sm_scale: float) -> torch.Tensor:
    """Attention of q float32 [B, HQ, 128] over the 16-token pages listed in
    pages int64 [B, KV, n] (page p = tokens 16p .. 16p + 15 of the cache)."""
    B, KV, G = prep["kw"].shape[:3]
    n = pages.shape[-1]
    heads = torch.arange(KV)[:, None]
    offs = torch.arange(16)
    outs = []
    for b in range(B):
        g, m = pages[b] // 2, pages[b] % 2                                    # [KV, n]
        kw = prep["kw"][b].view(KV, G, 2, 16, 16)[heads, g, m]               # [KV, n, 16 t, 16 w]
        k = _unpack(kw) * prep["ks"][b][heads, g] + prep["kz"][b][heads, g]  # [KV, n, 16, 128]
        tok = (pages[b].unsqueeze(-1) * 16 + offs).reshape(KV, n * 16)      # [KV, 16 n]
        vw = prep["vw"][b][heads, tok]                                       # [KV, 16 n, 16]
        v = (_unpack(vw).unflatten(-1, (4, 32)) * prep["vs"][b][heads, tok] +
             prep["vz"][b][heads, tok]).flatten(-2)
        o = torch.nn.functional.scaled_dot_product_attention(q[b].unsqueeze(1), k.reshape(KV, n * 16, 128), v,
                                                             scale=sm_scale, enable_gqa=True)
        outs.append(o.squeeze(1))
    return torch.stack(outs)


def c3_step(q: torch.Tensor, prep: dict, n_sel: int, sm_scale: float):
    """One C3 decode step: (selected pages [B, KV, n_sel], output [B, HQ, 128])."""
    sel = torch.topk(quest_scores(prep), n_sel, dim=-1).indices.sort(dim=-1).values
    return sel, sparse_attention(q, prep, sel, sm_scale)


# ---- C4: RaBitQ 1-bit search (see oracle/rabitq.py for the definitions) ----
#
#   * rotation y = (x * sigma) H with the Sylvester Hadamard matrix, codes
#     bit b of byte j = (y[8j + b] >= 0), norm = ||x||, corr = ||y|| sqrt(D) /
#     sum |y| (PC:1130-1195 with one SRHT round);
#   * estimate nk ck nq cq (D - 2 popc(xq ^ xk)) / D, the popcount taken on
#     64-bit words by the SWAR bit count;
#   * torch.topk of the estimates, then the exact fp32 dot of the candidates.

def _hadamard(d: int = 128) -> torch.Tensor:
    h = torch.ones(1, 1)
    while h.shape[0] < d:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return h


_M1, _M2, _M4 = 0x5555555555555555, 0x3333333333333333, 0x0F0F0F0F0F0F0F0F


def _popc64(v: torch.Tensor) -> torch.Tensor:
    """Bit count of int64 words (two's complement bits)."""
    v = v - ((v >> 1) & _M1)
    v = (v & _M2) + ((v >> 2) & _M2)
    v = (v + (v >> 4)) & _M4
    v = v + (v >> 8)
    v = v + (v >> 16)
    v = v + (v >> 32)
    return v & 0x7F


def prepare_c4(keys_f16: np.ndarray, codes: np.ndarray, fac_f16: np.ndarray, signs: np.ndarray) -> dict:
    """keys fp16 bits [N, 128], codes uint8 [N, 16], factors fp16 bits [N, 2]."""
    return {"keys": torch.from_numpy(f16_to_f32(keys_f16)),
            "codes": torch.from_numpy(np.ascontiguousarray(codes).view(np.int64)),     # [N, 2]
            "fk": torch.from_numpy(f16_to_f32(fac_f16)).prod(-1),
            "signs": torch.from_numpy(np.asarray(signs, np.float32)), "H": _hadamard()}


def c4_search(q: torch.Tensor, prep: dict, topk: int, q_block: int = 8):
    """q float32 [Q, 128] -> (candidates [Q, topk], exact scores [Q, topk])."""
    y = (q * prep["signs"]) @ prep["H"]
    bits = (y >= 0).to(torch.int64).view(-1, 16, 8)
    cq = (bits << torch.arange(8)).sum(-1).to(torch.uint8).contiguous().view(torch.int64)   # [Q, 2]
    # the query factors rounded to fp16, as the key factors are stored
    f16 = lambda t: t.to(torch.float16).to(torch.float32)
    fq = f16(q.norm(dim=-1)) * f16(y.norm(dim=-1) * math.sqrt(128.0) / y.abs().sum(-1))
    cands = []
    for i in range(0, q.shape[0], q_block):
        x = cq[i:i + q_block, None, :] ^ prep["codes"][None]                  # [q, N, 2]
        pc = _popc64(x).sum(-1)
        est = fq[i:i + q_block, None] * prep["fk"][None] * (128 - 2 * pc).to(torch.float32) / 128.0
        cands.append(torch.topk(est, topk, dim=-1).indices)
    cand = torch.cat(cands)
    exact = (q[:, None, :] * prep["keys"][cand]).sum(-1)
    return cand, exact
