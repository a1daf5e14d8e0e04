"""KIVI 4-bit quantize / pack / dequant and quantized decode attention (oracle).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Two storage formats are restated here.

Format R -- the reference's production K cache (S:646-744, S:1965-2157):
  packed_K   int32 [bs, kv, n_chunks, 16, g]  chunk-major; word (c, p, t) holds
             the 4-bit codes of channels 8p..8p+7 of token c*g+t, channel 8p+j
             in bits [4j, 4j+4) (quant_pack.py:124-141, transposed at S:2017).
  chunk_min / chunk_max  bf16 [bs, kv, n_chunks, 128]  (S:2119-2143)
  codes = rne(clamp(bf16(bf16(K - mn) / max(bf16(bf16(mx - mn) / 15),
                                            bf16(1e-8))), 0, 15))  (S:2003-2009)

Format Q -- the north-star 4-bit K *and* V cache with fp16 scale/zero
Codes follow the same ladder (K: per channel over
groups of 32 tokens; V: per token over groups of 32 channels); scale and zero
are the bf16 ladder's ``scale`` and ``mn`` converted to fp16 (RNE).  The word
and metadata order is chosen so that the gfx950 decode kernel's MFMA operands
need no cross-lane movement:

  k_codes  int32 [bs, kv, G, 512]  word m*256 + l*4 + s (l = 16g + c, g, c < 4, 16)
           holds the codes of channels 8p..8p+7 of token 32G + 16m + c, p = 4s + g,
           channel 8p+j in bits [4j, 4j+4)  (the reference's nibble packing)
  k_meta   fp16  [bs, kv, G, 16, 2, 8] [..., p, 0, s] = scale of channel
           8p + KSLOT[s], [..., p, 1, s] = zero (min) of that channel,
           KSLOT = (0, 4, 1, 5, 2, 6, 3, 7)
  v_codes  int32 [bs, kv, G, 512]  word m*256 + l*4 + P (l = 16g + c, half m,
           channel pair P) holds channels d = 32P + 2c and d + 1 of tokens
           32G + 16m + 4g + i: nibble n is token i = n//4 + 2(n%2) of channel
           d + (n//2)%2, i.e. nibbles (0, 4, 1, 5) = channel d, tokens
           (0, 1, 2, 3), nibbles (2, 6, 3, 7) = channel d + 1
  v_meta   fp16  [bs, kv, G, 2, 4, 4, 2, 4] [..., m, gd, r, 0, i] = scale of
           token 32G + 16m + 4r + i for channel group gd (channels
           32gd..32gd+31), [..., 1, i] = zero
Word l*4 + s of each 1 KiB block is what MFMA lane l of the decode kernel
consumes, so a lane's operands are contiguous 16-byte reads.  Each 16-token
half m of a group (one Quest page) has its own K code block (words m*256..),
V code block and 256-byte V metadata block; only the 512-byte K metadata is
shared by the two halves, so one page reads 2816 of the record's 5120 bytes.
The V-MFMA's k-slice of lane group g is tokens TAU[g] = (4g..4g+3,
16+4g..16+4g+3) -- where the K-MFMA leaves those scores -- so the decode
kernel takes the half-0 word for its elements 0-3 and the half-1 word for
4-7.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .numerics import BF16_1EM8, bf16r, f16_bits, f16_to_f32, f32

LEVELS = 15
GROUP_Q = 32                       # Format Q: tokens per K group / tile
KSLOT = np.array([0, 4, 1, 5, 2, 6, 3, 7])
TAU = np.array([[4 * r + e if e < 4 else 16 + 4 * r + (e - 4) for e in range(8)]
                for r in range(4)])
VNIB_TOK = np.array([n // 4 + 2 * (n % 2) for n in range(8)])   # token i of nibble n
VNIB_CH = np.array([(n // 2) % 2 for n in range(8)])            # channel d + VNIB_CH[n]


# ---------------------------------------------------------------------------
# The bf16 quantisation ladder
# ---------------------------------------------------------------------------
def kivi_scale(mn: np.ndarray, mx: np.ndarray, levels: int = LEVELS) -> np.ndarray:
    """Raw bf16 scale = bf16(bf16(mx - mn) / levels)  (quant_pack.py:51-65, S:2003)."""
    diff = bf16r(f32(mx) - f32(mn))
    return bf16r(diff / np.float32(levels))


def kivi_codes(x: np.ndarray, mn: np.ndarray, mx: np.ndarray,
               levels: int = LEVELS) -> np.ndarray:
    """Integer codes from the bf16 ladder (S:2003-2009; quant_pack.py:112-121).

    ``x``, ``mn``, ``mx`` hold bf16 values (float32 arrays) and broadcast.
    Every op is an IEEE float32 op followed by RNE to bf16, as torch does for
    bf16 tensors; ``clamp(min=1e-8)`` compares against bf16(1e-8); ``round``
    is half-to-even.
    """
    scale = kivi_scale(mn, mx, levels)
    safe = np.maximum(scale, BF16_1EM8)
    d = bf16r(f32(x) - f32(mn))
    qv = bf16r(d / safe)
    qv = np.clip(qv, np.float32(0.0), np.float32(levels))
    return np.rint(qv).astype(np.int32)


def pack_last_dim(codes: np.ndarray, bits: int = 4) -> np.ndarray:
    """word[p] = sum_j code[8p+j] << (bits*j) as int32  (quant_pack.py:124-141)."""
    fpi = 32 // bits
    c = np.asarray(codes, dtype=np.uint64)
    shp = c.shape[:-1] + (c.shape[-1] // fpi, fpi)
    c = c.reshape(shp)
    shifts = (np.arange(fpi, dtype=np.uint64) * np.uint64(bits))
    w = (c << shifts).sum(axis=-1) & np.uint64(0xFFFFFFFF)
    return w.astype(np.uint32).view(np.int32)


def unpack_last_dim(packed: np.ndarray, bits: int = 4) -> np.ndarray:
    """Inverse of ``pack_last_dim`` (quant_pack.py:166-174)."""
    fpi = 32 // bits
    u = np.asarray(packed).view(np.uint32).astype(np.uint64)
    shifts = (np.arange(fpi, dtype=np.uint64) * np.uint64(bits))
    c = (u[..., None] >> shifts) & np.uint64((1 << bits) - 1)
    return c.reshape(u.shape[:-1] + (u.shape[-1] * fpi,)).astype(np.int32)


# ---------------------------------------------------------------------------
# Format R: reference chunk-major K pack (S:1965-2157)
# ---------------------------------------------------------------------------
def chunk_minmax_mean(k_chunked: np.ndarray):
    """Per chunk / channel amin, amax and mean (S:2133-2135).

    ``k_chunked`` [..., n_chunks, g, D] bf16 values.  The mean is the
    canonical sequential float32 sum over the g tokens, divided by g and
    rounded to bf16 (torch's bf16 ``mean`` accumulates in float32; its
    reduction order is unspecified, this order is the one the build uses).
    """
    mn = k_chunked.min(axis=-2)
    mx = k_chunked.max(axis=-2)
    acc = np.zeros(k_chunked.shape[:-2] + k_chunked.shape[-1:], dtype=np.float32)
    for t in range(k_chunked.shape[-2]):
        acc = (acc + k_chunked[..., t, :]).astype(np.float32)
    mean = bf16r(acc / np.float32(k_chunked.shape[-2]))
    return mn, mx, mean


def pack_chunks_ref(k_chunked: np.ndarray, mn: np.ndarray, mx: np.ndarray) -> np.ndarray:
    """KIVI-encode chunks into the chunk-major layout (S:1997-2020).

    k_chunked [..., n_chunks, g, 128]; mn/mx [..., n_chunks, 128]
    returns int32 [..., n_chunks, 16, g].
    """
    codes = kivi_codes(k_chunked, mn[..., None, :], mx[..., None, :])
    packed = pack_last_dim(codes)                      # [..., n_chunks, g, 16]
    return np.ascontiguousarray(np.swapaxes(packed, -1, -2))


def encode_chunks_ref(keys: np.ndarray, g: int):
    """Full-chunk encode of a chunk-aligned K run (S:2119-2143).

    keys [bs, kv, n_tok, 128] bf16 values; n_tok // g chunks are encoded.
    Returns (chunk_min, chunk_max, chunk_centroid, packed_K).
    """
    bs, kv, n, d = keys.shape
    nc = n // g
    kc = keys[:, :, :nc * g].reshape(bs, kv, nc, g, d)
    mn, mx, mean = chunk_minmax_mean(kc)
    return mn, mx, mean, pack_chunks_ref(kc, mn, mx)


def dequant_ref(packed: np.ndarray, mn: np.ndarray, mx: np.ndarray) -> np.ndarray:
    """bf16(bf16(code * scale) + mn) with the raw (unclamped) scale (quant_pack.py:177-198).

    packed [..., n_chunks, 16, g] -> K_hat [..., n_chunks, g, 128] bf16 values.
    """
    codes = unpack_last_dim(np.swapaxes(packed, -1, -2)).astype(np.float32)
    scale = kivi_scale(mn, mx)[..., None, :]
    return bf16r(bf16r(codes * scale) + mn[..., None, :])


# ---------------------------------------------------------------------------
# Format Q: north-star 4-bit K and V cache with fp16 scale/zero
# ---------------------------------------------------------------------------
@dataclass
class Kivi4Cache:
    k_codes: np.ndarray   # int32  [bs, kv, G, 512] (lane order)
    k_meta: np.ndarray    # uint16 (fp16 bits) [bs, kv, G, 16, 2, 8]
    v_codes: np.ndarray   # int32  [bs, kv, G, 512] (lane order)
    v_meta: np.ndarray    # uint16 (fp16 bits) [bs, kv, G, 2, 4, 4, 2, 4]

    @property
    def n_groups(self) -> int:
        return self.k_codes.shape[2]


def k_words_to_lane_order(words: np.ndarray) -> np.ndarray:
    """[.., G, 16 (p), 32 (t)] chunk-major words -> [.., G, 512] lane order."""
    sh = words.shape[:-2]
    w = words.reshape(sh + (4, 4, 2, 16))                  # p = 4s + g, t = 16m + c
    w = np.moveaxis(w, (-4, -3, -2, -1), (-1, -3, -4, -2))  # -> [m, g, c, s]
    return np.ascontiguousarray(w).reshape(sh + (512,))


def k_words_from_lane_order(words: np.ndarray) -> np.ndarray:
    sh = words.shape[:-1]
    w = words.reshape(sh + (2, 4, 16, 4))                   # [m, g, c, s]
    w = np.moveaxis(w, (-4, -3, -2, -1), (-2, -3, -1, -4))  # -> [s, g, m, c]
    return np.ascontiguousarray(w).reshape(sh + (16, 32))


def v_codes_to_words(vc: np.ndarray) -> np.ndarray:
    """V codes [.., 32 (token), 128 (channel)] of a group -> [.., 512] int32 words."""
    sh = vc.shape[:-2]
    x = vc.astype(np.uint64).reshape(sh + (2, 4, 4, 4, 16, 2))   # [m, g, i, P, c, jp]
    words = np.zeros(sh + (2, 4, 16, 4), dtype=np.uint64)        # [m, g, c, P]
    for n in range(8):
        nib = x[..., VNIB_TOK[n], :, :, VNIB_CH[n]]               # [m, g, P, c]
        words |= np.swapaxes(nib, -1, -2) << np.uint64(4 * n)
    return words.astype(np.uint32).view(np.int32).reshape(sh + (512,))


def v_words_to_codes(words: np.ndarray) -> np.ndarray:
    """Inverse of v_codes_to_words: [.., 512] int32 -> codes [.., 32, 128] uint8."""
    sh = words.shape[:-1]
    w = words.view(np.uint32).astype(np.uint64).reshape(sh + (2, 4, 16, 4))   # [m, g, c, P]
    vc = np.empty(sh + (2, 4, 4, 4, 16, 2), dtype=np.uint8)                  # [m, g, i, P, c, jp]
    for n in range(8):
        nib = ((w >> np.uint64(4 * n)) & np.uint64(15)).astype(np.uint8)
        vc[..., VNIB_TOK[n], :, :, VNIB_CH[n]] = np.swapaxes(nib, -1, -2)
    return vc.reshape(sh + (32, 128))


def quantize_kivi4(k: np.ndarray, v: np.ndarray) -> Kivi4Cache:
    """Quantize G*32 tokens of K and V into Format Q.

    k, v [bs, kv, n_tok, 128] bf16 values; n_tok must be a multiple of 32.
    """
    bs, kv, n, d = k.shape
    assert d == 128 and n % GROUP_Q == 0
    ng = n // GROUP_Q
    # ---- K: per channel, groups of 32 tokens ----
    kg = k.reshape(bs, kv, ng, GROUP_Q, d)
    kmn = kg.min(axis=3)
    kmx = kg.max(axis=3)
    kc = kivi_codes(kg, kmn[:, :, :, None, :], kmx[:, :, :, None, :])   # [.., ng, 32, 128]
    k_codes = k_words_to_lane_order(np.swapaxes(pack_last_dim(kc), -1, -2))
    ksc = kivi_scale(kmn, kmx)                                          # [.., ng, 128]
    chan = (np.arange(16)[:, None] * 8 + KSLOT[None, :])                # [16, 8]
    k_meta = np.empty((bs, kv, ng, 16, 2, 8), dtype=np.uint16)
    k_meta[..., 0, :] = f16_bits(ksc[..., chan])
    k_meta[..., 1, :] = f16_bits(kmn[..., chan])
    # ---- V: per token, groups of 32 channels ----
    vg = v.reshape(bs, kv, n, 4, 32)
    vmn = vg.min(axis=4)
    vmx = vg.max(axis=4)
    vc = kivi_codes(vg, vmn[..., None], vmx[..., None]).reshape(bs, kv, ng, GROUP_Q, d)
    v_codes = v_codes_to_words(vc)
    # v_meta[..., m, gd, r, 0, i] = scale of token 16m + 4r + i, channel group gd
    vsc = kivi_scale(vmn, vmx).reshape(bs, kv, ng, 2, 4, 4, 4)        # [.., m, r, i, gd]
    vmn_g = vmn.reshape(bs, kv, ng, 2, 4, 4, 4)
    v_meta = np.empty((bs, kv, ng, 2, 4, 4, 2, 4), dtype=np.uint16)
    v_meta[..., 0, :] = f16_bits(np.moveaxis(vsc, -1, -3))
    v_meta[..., 1, :] = f16_bits(np.moveaxis(vmn_g, -1, -3))
    return Kivi4Cache(k_codes, k_meta, v_codes, v_meta)


def kivi4_codes_and_meta(k: np.ndarray, v: np.ndarray):
    """Logical (unpermuted) view of Format Q: codes [.., n, 128] and fp32 scale/zero.

    Returns (k_code, k_scale[.., G, 128], k_zero, v_code, v_scale[.., n, 4], v_zero).
    """
    bs, kv, n, d = k.shape
    ng = n // GROUP_Q
    kg = k.reshape(bs, kv, ng, GROUP_Q, d)
    kmn = kg.min(axis=3)
    kmx = kg.max(axis=3)
    kc = kivi_codes(kg, kmn[:, :, :, None, :], kmx[:, :, :, None, :]).reshape(bs, kv, n, d)
    vg = v.reshape(bs, kv, n, 4, 32)
    vmn = vg.min(axis=4)
    vmx = vg.max(axis=4)
    vc = kivi_codes(vg, vmn[..., None], vmx[..., None]).reshape(bs, kv, n, d)
    return (kc, f16_to_f32(f16_bits(kivi_scale(kmn, kmx))), f16_to_f32(f16_bits(kmn)),
            vc, f16_to_f32(f16_bits(kivi_scale(vmn, vmx))), f16_to_f32(f16_bits(vmn)))


def dequant_kivi4(c: Kivi4Cache, dtype=np.float64):
    """Exact dequant code*scale + zero (no intermediate rounding) of Format Q.

    Returns K_hat, V_hat [bs, kv, G*32, 128] in ``dtype``.
    """
    bs, kv, ng = c.k_codes.shape[:3]
    # K
    kcodes = unpack_last_dim(np.swapaxes(k_words_from_lane_order(c.k_codes), -1, -2)).astype(dtype)
    kmeta = f16_to_f32(c.k_meta).astype(dtype)                               # [.., ng, 16, 2, 8]
    chan = (np.arange(16)[:, None] * 8 + KSLOT[None, :]).reshape(-1)
    ksc = np.empty((bs, kv, ng, 128), dtype=dtype)
    kzr = np.empty((bs, kv, ng, 128), dtype=dtype)
    ksc[..., chan] = kmeta[..., 0, :].reshape(bs, kv, ng, 128)
    kzr[..., chan] = kmeta[..., 1, :].reshape(bs, kv, ng, 128)
    k_hat = kcodes * ksc[:, :, :, None, :] + kzr[:, :, :, None, :]
    # V
    vcode = v_words_to_codes(c.v_codes).astype(dtype)                          # [.., ng, 32, 128]
    vmeta = f16_to_f32(c.v_meta).astype(dtype)                                # [.., ng, m, gd, r, 2, i]
    vsc = np.moveaxis(vmeta[..., 0, :], -3, -1).reshape(bs, kv, ng, GROUP_Q, 4)
    vzr = np.moveaxis(vmeta[..., 1, :], -3, -1).reshape(bs, kv, ng, GROUP_Q, 4)
    vsc = np.repeat(vsc, 32, axis=-1)
    vzr = np.repeat(vzr, 32, axis=-1)
    v_hat = vcode * vsc + vzr
    n = ng * GROUP_Q
    return k_hat.reshape(bs, kv, n, 128), v_hat.reshape(bs, kv, n, 128)


# ---------------------------------------------------------------------------
# Attention (textbook softmax; stands in for flash-attn 2.8.3's math at the
# S:1742-1747 call site, causal=False, GQA Hq/Hkv query heads per KV head)
# ---------------------------------------------------------------------------
def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, sm_scale: float,
              dtype=np.float64, return_lse: bool = False):
    """q [bs, Hq, D]; k, v [bs, Hkv, n, D] -> out [bs, Hq, D] (and lse [bs, Hq])."""
    bs, hq, d = q.shape
    hkv = k.shape[1]
    gqa = hq // hkv
    qq = q.astype(dtype).reshape(bs, hkv, gqa, d)
    s = np.einsum("bhgd,bhnd->bhgn", qq, k.astype(dtype)) * dtype(sm_scale)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(axis=-1, keepdims=True)
    o = np.einsum("bhgn,bhnd->bhgd", p, v.astype(dtype)) / l
    out = o.reshape(bs, hq, d)
    if return_lse:
        return out, (m + np.log(l)).reshape(bs, hq)
    return out


def kivi4_decode_attention(q, cache: Kivi4Cache, n_groups: int, k_res, v_res,
                           res_len: int, sm_scale: float, dtype=np.float64, return_lse: bool = False):
    """Decode attention over the first ``n_groups`` groups of a Format Q cache
    plus ``res_len`` full-precision residual tokens.

    q [bs, Hq, 128] (bf16 values); k_res / v_res [bs, Hkv, >=res_len, 128].
    With ``return_lse`` also the natural-log LSE [bs, Hq] of the scaled scores.
    """
    kh, vh = dequant_kivi4(Kivi4Cache(cache.k_codes[:, :, :n_groups],
                                      cache.k_meta[:, :, :n_groups],
                                      cache.v_codes[:, :, :n_groups],
                                      cache.v_meta[:, :, :n_groups]), dtype=dtype)
    k = np.concatenate([kh, k_res[:, :, :res_len].astype(dtype)], axis=2)
    v = np.concatenate([vh, v_res[:, :, :res_len].astype(dtype)], axis=2)
    return attention(q, k, v, sm_scale, dtype=dtype, return_lse=return_lse)


def kivi4_sparse_attention(q, cache: Kivi4Cache, n_groups: int, k_res, v_res, res_len: int,
                           pages: np.ndarray, sm_scale: float, dtype=np.float64, return_lse: bool = False):
    """Attention over the gathered tokens of the listed 16-token pages (page P =
    tokens 16P .. 16P+15 of the quantized region; ids outside [0, 2 n_groups)
    skipped, repeats kept) plus the residual window: the reference's
    gather -> flash_attn_with_kvcache(causal=False) (S:1723-1772).
    pages int [bs, Hkv, n_sel] -> out [bs, Hq, 128] (and with ``return_lse``
    the natural-log LSE [bs, Hq]; -inf where nothing is attended)."""
    kh, vh = dequant_kivi4(Kivi4Cache(cache.k_codes[:, :, :n_groups],
                                      cache.k_meta[:, :, :n_groups],
                                      cache.v_codes[:, :, :n_groups],
                                      cache.v_meta[:, :, :n_groups]), dtype=dtype)
    bs, hq, d = q.shape
    kv = kh.shape[1]
    gqa = hq // kv
    out = np.zeros((bs, hq, d), dtype=dtype)
    lse = np.full((bs, hq), -np.inf, dtype=dtype)
    for b in range(bs):
        for h in range(kv):
            p = np.asarray(pages[b, h]).astype(np.int64)
            p = p[(p >= 0) & (p < 2 * n_groups)]
            tok = (p[:, None] * 16 + np.arange(16)).reshape(-1)
            k = np.concatenate([kh[b, h, tok], k_res[b, h, :res_len].astype(dtype)], axis=0)
            v = np.concatenate([vh[b, h, tok], v_res[b, h, :res_len].astype(dtype)], axis=0)
            if k.shape[0] == 0:
                continue
            o, l = attention(q[b:b + 1, h * gqa:(h + 1) * gqa], k[None, None], v[None, None], sm_scale,
                             dtype=dtype, return_lse=True)
            out[b, h * gqa:(h + 1) * gqa] = o[0]
            lse[b, h * gqa:(h + 1) * gqa] = l[0]
    return (out, lse) if return_lse else out


def kivi4_token_attention(q, cache: Kivi4Cache, n_groups: int, k_rows, v_rows, toks: np.ndarray,
                          tail_row0: int, n_tail: int, near_row0: int, near_len: int, sm_scale: float,
                          dtype=np.float64, return_lse: bool = False):
    """Attention over a token list plus contiguous bf16 rows: the reference's
    gather of sink + local + the selected tokens followed by
    flash_attn_with_kvcache(causal=False) (S:1723-1772), with the retrieval
    zone's complete 32-token groups in Format Q.

    For (b, h), the listed ids in order: an id in [0, 32 n_groups) is that
    token of the Format Q records (exact dequant), an id in [32 n_groups,
    32 n_groups + n_tail) is the bf16 row tail_row0 + (id - 32 n_groups) of
    k_rows / v_rows [bs, Hkv, n_rows, 128]; other ids are skipped and a repeated
    id is attended again; then rows [near_row0, near_row0 + near_len).
    toks int [bs, Hkv, n_tok] -> out [bs, Hq, 128] (and the natural-log LSE
    [bs, Hq], -inf where nothing is attended)."""
    kh, vh = dequant_kivi4(Kivi4Cache(cache.k_codes[:, :, :n_groups], cache.k_meta[:, :, :n_groups],
                                      cache.v_codes[:, :, :n_groups], cache.v_meta[:, :, :n_groups]), dtype=dtype)
    bs, hq, d = q.shape
    kv = k_rows.shape[1]
    gqa = hq // kv
    q_end = 32 * n_groups
    out = np.zeros((bs, hq, d), dtype=dtype)
    lse = np.full((bs, hq), -np.inf, dtype=dtype)
    near = slice(near_row0, near_row0 + near_len)
    for b in range(bs):
        for h in range(kv):
            ids = np.asarray(toks[b, h]).astype(np.int64)
            ks, vs = [], []
            for t in ids:
                if 0 <= t < q_end:
                    ks.append(kh[b, h, t])
                    vs.append(vh[b, h, t])
                elif q_end <= t < q_end + n_tail:
                    ks.append(k_rows[b, h, tail_row0 + t - q_end].astype(dtype))
                    vs.append(v_rows[b, h, tail_row0 + t - q_end].astype(dtype))
            k = np.concatenate([np.array(ks, dtype=dtype).reshape(-1, d), k_rows[b, h, near].astype(dtype)], axis=0)
            v = np.concatenate([np.array(vs, dtype=dtype).reshape(-1, d), v_rows[b, h, near].astype(dtype)], axis=0)
            if k.shape[0] == 0:
                continue
            o, l = attention(q[b:b + 1, h * gqa:(h + 1) * gqa], k[None, None], v[None, None], sm_scale,
                             dtype=dtype, return_lse=True)
            out[b, h * gqa:(h + 1) * gqa] = o[0]
            lse[b, h * gqa:(h + 1) * gqa] = l[0]
    return (out, lse) if return_lse else out


def lse_merge(out_a, lse_a, out_b, lse_b, dtype=np.float64):
    """lse_merge_torch (Z/cache_hub/lse_merge/lse_merge.py:79-119):
    out_* [bs, heads, dim], lse_* [bs, heads] (natural log)."""
    la, lb = lse_a.astype(dtype), lse_b.astype(dtype)
    m = np.maximum(la, lb)
    wa, wb = np.exp(la - m), np.exp(lb - m)
    return ((wa[..., None] * out_a.astype(dtype) + wb[..., None] * out_b.astype(dtype))
            / (wa + wb)[..., None])
