"""PyTorch-CPU restatement of the C2 decode step: the CPU baseline of
``bench.py`` (its ``cpu_baseline`` leg).

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
