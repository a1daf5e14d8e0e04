"""ParisKV-compatible 4-bit RaBitQ codes on gfx950 (1-bit sign + 3-bit
magnitude per rotated dimension, bf16 block weights) and their rerank.

Mirrors the reference's ParisKV RaBitQ pieces, with the same names, shapes,
dtypes and error behaviour (PC = Z/cache_hub/polar_cache.py):

* ``MultiDimBlockQuantizer`` (PC:49-126): the seeded SRHT sign vector and the
  sign codebook JSON (``{"config": {d, m, K_r, K_omega, ...},
  "angular_signs": [[+-1] * m] * K_omega}``, e.g.
  ``turboquant/codebooks/codebook_d128_m8_Kr1_Kw256_rabitq_sign.json``);
* ``magnitude_levels`` (PC:266-270, or a ``codebooks/magnitude_levels_m8*.json``
  file): 7 thresholds and 8 centers as bf16;
* ``batch_encode`` (PC:1130-1195, with ``_pack_4bit_codes`` PC:1067-1084):
  codebook uint8 [bs, kv, 16, seq], block_weight bf16 [bs, kv, 16, seq],
  packed_4bit uint8 [bs, kv, 16, seq, 4];
* ``encode_query_blocks`` (``_encode_query_blocks``, PC:1108-1124);
* ``partial_rerank_cuda`` / ``partial_rerank_scores_cuda``
  (Z/cache_hub/rerank/rerank.py:352-440, kernel rerank.cu:52-143);
* ``rabitq_rerank_topk``: the rerank + ``torch.topk`` + gather of
  ``get_candidate_cache_with_rabitq_rerank`` (PC:1750-1825), as one score
  launch and one top-k launch.  The set equals the reference's (ties to the
  earlier candidate position); it comes in increasing candidate position.

Every value is rounded to bf16 where the reference's torch ops round, so codes,
weights, query blocks and scores equal the reference's bit for bit (the
reference's fp32 reductions of the key norm are ordered by the kernel; the
committed reference vectors agree).
"""
from __future__ import annotations

import json

import torch

from . import topk as _topk_mod
from ._lib import check, device_stream, lib, ptr, require_gpu, stream_of

HEAD_DIM = 128
DEFAULT_SRHT_ROUNDS = 1  # PC:35
MAG_THRESHOLDS = [0.0843, 0.1698, 0.2578, 0.3499, 0.4487, 0.5585, 0.6901]  # PC:267
MAG_CENTERS = [0.0420, 0.1266, 0.2130, 0.3025, 0.3973, 0.5001, 0.6169, 0.7633]  # PC:269


class MultiDimBlockQuantizer:
    """The reference quantizer's state (PC:49-126): d-dim vectors in B = d / m
    blocks, ``srht_diagonal_signs`` (bf16 +-1, drawn from torch's seeded RNG
    on ``device`` with the caller's RNG state restored) and the sign codebook
    ``V_omega_gpu`` (bf16 +-1 [K_omega, m]) loaded from ``codebook_path``."""

    def __init__(self, d, m, K_r, K_omega, codebook_path, seed=42, device=None):
        assert d % m == 0, f"total dimension {d} must be divisible by the block dimension {m}"
        if not torch.cuda.is_available():
            raise RuntimeError("no GPU available: this quantizer runs on the GPU only")
        self.d, self.m, self.B = d, m, d // m
        self.K_r, self.K_omega, self.K_total = K_r, K_omega, K_r * K_omega
        self.seed = seed
        if device is None:
            device = torch.device("cuda:0")
        elif isinstance(device, str):
            device = torch.device(device)
        rng_state = torch.get_rng_state()
        cuda_rng_state = torch.cuda.get_rng_state()
        torch.manual_seed(self.seed)
        self.srht_diagonal_signs = []
        for _ in range(DEFAULT_SRHT_ROUNDS):
            signs = torch.randint(0, 2, (self.d,), device=device, dtype=torch.bfloat16) * 2 - 1
            self.srht_diagonal_signs.append(signs)
        torch.set_rng_state(rng_state)
        torch.cuda.set_rng_state(cuda_rng_state)
        try:
            with open(codebook_path, "r") as f:
                codebook = json.load(f)
            config = codebook["config"]
            if (config["d"] != self.d or config["m"] != self.m or config["K_r"] != self.K_r
                    or config["K_omega"] != self.K_omega):
                raise ValueError(
                    f"codebook parameters do not match: expected d={self.d}, m={self.m}, K_r={self.K_r}, "
                    f"K_omega={self.K_omega}; got d={config['d']}, m={config['m']}, K_r={config['K_r']}, "
                    f"K_omega={config['K_omega']}")
            raw = codebook["angular_signs"] if "angular_signs" in codebook else codebook["angular_centers"]
            vals = torch.tensor(raw, dtype=torch.float32, device=device)
            self.V_omega_gpu = torch.where(vals >= 0, 1.0, -1.0).to(torch.bfloat16)
        except FileNotFoundError:
            raise FileNotFoundError(f"codebook file not found: {codebook_path}")
        except (KeyError, json.JSONDecodeError) as e:
            raise ValueError(f"malformed codebook file: {e}")


def magnitude_levels(path=None, device="cuda"):
    """(thresholds bf16 [7], centers bf16 [8]): PC:266-270, or the
    ``thresholds`` / ``centers`` of a magnitude-levels JSON file."""
    thr, ctr = MAG_THRESHOLDS, MAG_CENTERS
    if path is not None:
        with open(path, "r") as f:
            lv = json.load(f)
        thr, ctr = lv["thresholds"], lv["centers"]
        if len(thr) != 7 or len(ctr) != 8:
            raise ValueError(f"8-level magnitude file expected (7 thresholds, 8 centers); got {len(thr)}, {len(ctr)}")
    return (torch.tensor(thr, dtype=torch.bfloat16, device=device).contiguous(),
            torch.tensor(ctr, dtype=torch.bfloat16, device=device).contiguous())


def _signs16(signs: torch.Tensor) -> torch.Tensor:
    if signs.dtype != torch.bfloat16 or signs.shape != (HEAD_DIM,) or not signs.is_contiguous() \
            or signs.data_ptr() % 16:
        signs = signs.to(torch.bfloat16).contiguous().clone()
    return signs


def _rows16(x: torch.Tensor) -> torch.Tensor:
    """bf16, last dim contiguous, rows and base 16-byte aligned."""
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    if x.stride(-1) != 1 or x.data_ptr() % 16 or any(s % 8 for s in x.stride()[:-1]):
        x = x.contiguous()
    return x


def encode_into(Y: torch.Tensor, signs: torch.Tensor, mag_thresholds: torch.Tensor, mag_centers: torch.Tensor,
                codebook: torch.Tensor, block_weight: torch.Tensor, packed_4bit: torch.Tensor, t0: int = 0) -> None:
    """Encode keys Y [bs, kv, n, 128] into token positions t0 .. t0 + n - 1 of
    codebook uint8 [bs, kv, 16, cap], block_weight bf16 [bs, kv, 16, cap] and
    packed_4bit uint8 [bs, kv, 16, cap, 4] (unit token stride in each)."""
    require_gpu(Y, signs, mag_thresholds, mag_centers, codebook, block_weight, packed_4bit)
    assert Y.dim() == 4 and Y.shape[-1] == HEAD_DIM, f"keys must be [bs, kv, n, 128]; got {tuple(Y.shape)}"
    bs, kv, n, _ = Y.shape
    cap = codebook.shape[-1]
    assert codebook.dtype == torch.uint8 and block_weight.dtype == torch.bfloat16 and packed_4bit.dtype == torch.uint8
    assert codebook.shape == (bs, kv, 16, cap) and block_weight.shape == (bs, kv, 16, cap) \
        and packed_4bit.shape == (bs, kv, 16, cap, 4), "output shapes must be [bs, kv, 16, cap] (and [..., 4])"
    assert codebook.stride(-1) == 1 and block_weight.stride(-1) == 1 and packed_4bit.stride(-1) == 1 \
        and packed_4bit.stride(-2) == 4, "outputs need a unit token stride (4 bytes for packed_4bit)"
    assert all(s % 4 == 0 for s in packed_4bit.stride()[:3]), "packed_4bit strides must be whole 4-byte words"
    assert 0 <= t0 and t0 + n <= cap, f"tokens {t0}..{t0 + n} exceed the capacity {cap}"
    assert mag_thresholds.dtype == torch.bfloat16 and mag_thresholds.numel() == 7 and mag_thresholds.is_contiguous()
    assert mag_centers.dtype == torch.bfloat16 and mag_centers.numel() == 8 and mag_centers.is_contiguous()
    Y = _rows16(Y)
    s = _signs16(signs)
    ps = packed_4bit.stride()
    check(lib().zkv_rabitq4_encode(
        ptr(Y), Y.stride(0), Y.stride(1), Y.stride(2), bs, kv, n, ptr(s), ptr(mag_thresholds), ptr(mag_centers),
        ptr(codebook), codebook.stride(0), codebook.stride(1), codebook.stride(2),
        ptr(packed_4bit), ps[0] // 4, ps[1] // 4, ps[2] // 4,
        ptr(block_weight), block_weight.stride(0), block_weight.stride(1), block_weight.stride(2), int(t0),
        stream_of(Y)))


def batch_encode(Y: torch.Tensor, signs: torch.Tensor, mag_thresholds: torch.Tensor = None,
                 mag_centers: torch.Tensor = None, return_rabitq: bool = True):
    """PC:1130-1195: Y [bs, kv, seq, 128] -> (codebook uint8 [bs, kv, 16, seq],
    block_weight bf16 [bs, kv, 16, seq] or None, packed_4bit uint8
    [bs, kv, 16, seq, 4] or None)."""
    require_gpu(Y)
    if mag_thresholds is None or mag_centers is None:
        mag_thresholds, mag_centers = magnitude_levels(device=Y.device)
    bs, kv, seq, _ = Y.shape
    codebook = torch.empty(bs, kv, 16, seq, dtype=torch.uint8, device=Y.device)
    block_weight = torch.empty(bs, kv, 16, seq, dtype=torch.bfloat16, device=Y.device)
    packed = torch.empty(bs, kv, 16, seq, 4, dtype=torch.uint8, device=Y.device)
    encode_into(Y, signs, mag_thresholds, mag_centers, codebook, block_weight, packed, 0)
    if not return_rabitq:
        return codebook, None, None
    return codebook, block_weight, packed


def encode_query_blocks(query: torch.Tensor, signs: torch.Tensor):
    """PC:1108-1124: query [bs, kv, 128] -> (q_blocks bf16 [bs, kv, 16, 8],
    q_norm bf16 [bs, kv, 1])."""
    require_gpu(query, signs)
    assert query.shape[-1] == HEAD_DIM, f"query rows must be 128 wide; got {tuple(query.shape)}"
    lead = query.shape[:-1]
    q = _rows16(query.reshape(-1, HEAD_DIM))
    rows = q.shape[0]
    q_blocks = torch.empty(*lead, 16, 8, dtype=torch.bfloat16, device=query.device)
    q_norm = torch.empty(*lead, 1, dtype=torch.bfloat16, device=query.device)
    check(lib().zkv_rabitq4_encode_query(ptr(q), q.stride(0), rows, ptr(_signs16(signs)), ptr(q_blocks),
                                         ptr(q_norm), stream_of(q)))
    return q_blocks, q_norm


def _validate(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, B, m):
    """rerank.py:323-349, plus the layout this kernel reads."""
    bs, kv_heads, B_dim, kv_len, _ = key_4bit.shape
    assert B_dim == B, f"B mismatch: key_4bit has {B_dim}, got B={B}"
    assert m == 8, f"m must be 8, got {m}"
    assert B == 16, "only B = 16 is supported (rerank.cu:215-220)"
    assert coarse_indices.dtype == torch.int64, f"coarse_indices must be int64, got {coarse_indices.dtype}"
    assert coarse_indices.is_contiguous()
    assert key_4bit.dtype == torch.uint8 and key_4bit.stride(-1) == 1
    assert key_block_weight.dtype == torch.bfloat16 and key_block_weight.stride(-1) == 1
    assert all(s % 4 == 0 for s in key_4bit.stride()[:4]), "key_4bit strides must be whole 4-byte words"
    assert key_block_weight.shape == key_4bit.shape[:4], "key_block_weight must be [bs, kv, B, kv_len]"
    assert q_blocks.dtype == torch.bfloat16 and q_blocks.is_contiguous()
    assert q_blocks.shape == (bs, kv_heads, B, m), f"q_blocks must be [bs, kv, B, m]; got {tuple(q_blocks.shape)}"
    assert q_norm.is_contiguous() and q_norm.numel() == bs * kv_heads
    assert mag_centers.dtype == torch.bfloat16 and mag_centers.is_contiguous() and mag_centers.numel() == 8
    assert coarse_indices.shape[:2] == (bs, kv_heads)
    require_gpu(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers)
    return bs, kv_heads, kv_len


# Streamed-path workspace per (device, stream): [tensor, (bs, kv, kv_len) of
# the last call or None].  Its token flags are zero between calls of one
# shape (each call leaves them zero); they are zeroed again when the shape
# changes.  Calls on one stream run in order, so they never share the flags
# or token scores while another call's kernels still use them; calls on two
# streams get two workspaces.
_WS: dict = {}


def _flag_bytes(bs: int, kv: int, kv_len: int) -> int:
    """The flag prefix of the workspace (one byte per token, rows rounded up
    to 1024 tokens, the whole to 256 bytes)."""
    return (bs * kv * ((kv_len + 1023) // 1024) * 1024 + 255) // 256 * 256


def _rerank_workspace(device, bs: int, kv: int, kv_len: int):
    need = lib().zkv_rabitq4_rerank_workspace_size(bs, kv, kv_len)
    dev = torch.device(device)
    key = (dev, device_stream(dev))
    ent = _WS.get(key)
    if ent is None or ent[0].numel() < need:
        ent = [torch.zeros(max(need, 1 << 16), dtype=torch.uint8, device=dev), (bs, kv, kv_len)]
        _WS[key] = ent
    elif ent[1] != (bs, kv, kv_len):
        ent[0][:_flag_bytes(bs, kv, kv_len)].zero_()
        ent[1] = (bs, kv, kv_len)
    return ent


def _rerank(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, B, m,
            scores=None, scores_f32=None, v4b=None):
    if q_norm.dtype != torch.bfloat16:
        q_norm = q_norm.to(torch.bfloat16).contiguous()
    bs, kv, kv_len = _validate(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, B, m)
    C = coarse_indices.shape[-1]
    ks, ws = key_4bit.stride(), key_block_weight.stride()
    ent = _rerank_workspace(key_4bit.device, bs, kv, kv_len) if v4b is None and kv_len > 0 and C > 0 else None
    try:
        check(lib().zkv_rabitq4_rerank(
            ptr(coarse_indices), coarse_indices.stride(0), coarse_indices.stride(1), bs, kv, C,
            ptr(key_4bit), ks[0] // 4, ks[1] // 4, ks[2] // 4, ks[3] // 4, kv_len,
            ptr(key_block_weight), ws[0], ws[1], ws[2], ptr(q_blocks), ptr(q_norm), ptr(mag_centers),
            ptr(scores), ptr(scores_f32), ptr(v4b), None if ent is None else ptr(ent[0]),
            0 if ent is None else ent[0].numel(), stream_of(key_4bit)))
    except Exception:
        if ent is not None:
            ent[1] = None  # a failed call may leave bits set: zero before the next
        raise


def partial_rerank_cuda(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, B, m,
                        kernel=None):
    """rerank.py:352-400: (approx_scores bf16 [bs, kv, C], v4b bf16
    [bs, kv, B, C, m] the decoded 4-bit values).  ``kernel`` is accepted for
    the reference's signature and unused.  A candidate outside
    [0, kv_len) scores -inf and decodes to zeros."""
    bs, kv, C = coarse_indices.shape
    scores = torch.empty(bs, kv, C, dtype=torch.bfloat16, device=coarse_indices.device)
    v4b = torch.empty(bs, kv, B, C, m, dtype=torch.bfloat16, device=coarse_indices.device)
    _rerank(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, B, m, scores=scores, v4b=v4b)
    return scores, v4b


def partial_rerank_scores_cuda(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, B, m,
                               kernel=None):
    """rerank.py:402-440: approx_scores bf16 [bs, kv, C] only."""
    bs, kv, C = coarse_indices.shape
    scores = torch.empty(bs, kv, C, dtype=torch.bfloat16, device=coarse_indices.device)
    _rerank(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, B, m, scores=scores)
    return scores


def rabitq_rerank_topk(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, final_topk,
                       B=16, m=8, return_scores=False):
    """The rerank and top-k of get_candidate_cache_with_rabitq_rerank
    (PC:1750-1825): scores of the candidates, then the ``min(final_topk, C)``
    best as key indices [bs, kv, k] (ties to the earlier candidate position,
    in increasing candidate position).  With return_scores, also the bf16
    scores [bs, kv, C]."""
    bs, kv, C = coarse_indices.shape
    k = min(int(final_topk), C)
    if k <= 0:
        out = torch.empty(bs, kv, 0, dtype=torch.int64, device=coarse_indices.device)
        sc = torch.empty(bs, kv, C, dtype=torch.bfloat16, device=coarse_indices.device)
        return (out, sc) if return_scores else out
    f32 = torch.empty(bs, kv, C, dtype=torch.float32, device=coarse_indices.device)
    sc = torch.empty(bs, kv, C, dtype=torch.bfloat16, device=coarse_indices.device) if return_scores else None
    _rerank(coarse_indices, key_4bit, key_block_weight, q_blocks, q_norm, mag_centers, B, m, scores=sc,
            scores_f32=f32)
    out = torch.empty(bs, kv, k, dtype=torch.int64, device=coarse_indices.device)
    _topk_mod._topk(f32, k, out, lut=coarse_indices)
    return (out, sc) if return_scores else out
