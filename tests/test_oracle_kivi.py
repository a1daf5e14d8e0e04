"""Pins of the KIVI oracle (CPU).  See oracle/__init__.py PINNING."""
import numpy as np
import pytest
import torch

from oracle import kivi
from oracle import kivi as okivi
from oracle.numerics import BF16_1EM8, bf16_bits, bf16_to_f32, bf16r, f16_bits
from tests.helpers import gaussian_bf16


def test_bf16_round_matches_torch_on_all_bf16_neighbourhoods():
    hi = np.arange(1 << 16, dtype=np.uint32)
    hi = hi[((hi << 16) & 0x7F800000) != 0x7F800000]          # finite only
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], dtype=np.uint32)
    u = ((hi[:, None] << 16) | lows[None, :]).reshape(-1)
    x = u.view(np.float32)
    ours = bf16_bits(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_scale_division_equals_reciprocal_multiply_for_every_bf16():
    """torch on CUDA computes bf16 / python-scalar as x * fp32(1/15) (the
    reference's production path, S:2003); torch on CPU and this oracle divide.
    Both round to the same bf16 for every non-negative finite bf16 diff."""
    u = np.arange(0, 0x7F80, dtype=np.uint32)
    d = bf16_to_f32(u.astype(np.uint16))
    div = bf16_bits(d / np.float32(15.0))
    mul = bf16_bits(d * (np.float32(1.0) / np.float32(15.0)))
    assert np.array_equal(div, mul)


def _torch_ladder(K, mn, mx):
    """The reference's torch op sequence (S:2003-2009 / quant_pack.py:112-121) on CPU bf16."""
    scale = (mx - mn) / float(15)
    scale_safe = scale.clamp(min=1e-8)
    return ((K - mn) / scale_safe).clamp_(0.0, 15.0).round_().to(torch.int32)


@pytest.mark.parametrize("g", [8, 16, 32])
def test_kivi_codes_match_torch_bf16_ops(rng, g):
    k = gaussian_bf16(rng, (2, 3, 7 * g, 128), outlier_channels=4)
    k[0, 0, :g, 5] = k[0, 0, 0, 5]                 # one flat chunk/channel
    kc = k.reshape(2, 3, 7, g, 128)
    mn = kc.min(axis=3, keepdims=True)
    mx = kc.max(axis=3, keepdims=True)
    ours = kivi.kivi_codes(kc, mn, mx)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)
    ref = _torch_ladder(t(kc), t(mn), t(mx)).numpy()
    assert np.array_equal(ours, ref)
    assert ours.min() >= 0 and ours.max() <= 15
    assert np.all(ours[0, 0, 0, :, 5] == 0)        # flat group -> all zero codes
    # the maximum of every (non-flat) group/channel encodes to 15, the minimum to 0
    at_max = kc == mx
    assert np.all(ours[at_max & (mx != mn)] == 15)
    assert np.all(ours[kc == mn] == 0)


def test_per_token_ladder_matches_torch(rng):
    v = gaussian_bf16(rng, (2, 2, 40, 128), outlier_channels=2)
    vg = v.reshape(2, 2, 40, 4, 32)
    mn = vg.min(axis=4, keepdims=True)
    mx = vg.max(axis=4, keepdims=True)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)
    assert np.array_equal(kivi.kivi_codes(vg, mn, mx), _torch_ladder(t(vg), t(mn), t(mx)).numpy())


def test_clamp_constant_is_bf16_of_1e8():
    assert float(BF16_1EM8) == float(torch.tensor(1e-8, dtype=torch.bfloat16).float())


def test_pack_unpack_every_code_at_every_position():
    codes = np.zeros((16, 8, 8), dtype=np.int32)
    for val in range(16):
        for pos in range(8):
            codes[val, pos, pos] = val
    packed = kivi.pack_last_dim(codes)
    assert packed.shape == (16, 8, 1)
    for val in range(16):
        for pos in range(8):
            w = int(packed[val, pos, 0]) & 0xFFFFFFFF
            assert w == val << (4 * pos)
    assert np.array_equal(kivi.unpack_last_dim(packed), codes)
    # bit 31 set -> negative int32, exactly as torch's int32 sum (quant_pack.py:140)
    assert packed[15, 7, 0] < 0


def test_pack_matches_torch_shift_sum(rng):
    codes = rng.integers(0, 16, size=(3, 5, 128), dtype=np.int32)
    t = torch.from_numpy(codes).view(3, 5, 16, 8)
    shifts = torch.arange(8, dtype=torch.int32) * 4
    ref = (t << shifts).sum(dim=-1, dtype=torch.int32).numpy()
    assert np.array_equal(kivi.pack_last_dim(codes), ref)


def test_format_r_layout_is_chunk_major(rng):
    k = gaussian_bf16(rng, (1, 2, 48, 128))
    mn, mx, mean, packed = kivi.encode_chunks_ref(k, 16)
    assert packed.shape == (1, 2, 3, 16, 16)
    codes = kivi.kivi_codes(k.reshape(1, 2, 3, 16, 128), mn[:, :, :, None], mx[:, :, :, None])
    tok = kivi.pack_last_dim(codes)               # [.., chunk, token, p]
    assert np.array_equal(packed, np.swapaxes(tok, -1, -2))
    t = torch.from_numpy(k.reshape(1, 2, 3, 16, 128)).to(torch.bfloat16)
    assert np.array_equal(bf16_bits(mn), t.amin(dim=3).view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(bf16_bits(mx), t.amax(dim=3).view(torch.int16).numpy().view(np.uint16))
    # torch's bf16 mean agrees with the canonical sequential fp32 sum whenever the sum is exact
    ref_mean = t.mean(dim=3).float().numpy()
    assert np.max(np.abs(ref_mean - mean)) <= np.max(np.abs(mean)) * 2 ** -7


def test_dequant_ref_is_two_rounding_bf16_ladder(rng):
    k = gaussian_bf16(rng, (1, 1, 32, 128))
    mn, mx, _, packed = kivi.encode_chunks_ref(k, 16)
    kh = kivi.dequant_ref(packed, mn, mx)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)
    codes = kivi.unpack_last_dim(np.swapaxes(packed, -1, -2))
    scale = (t(mx) - t(mn)) / 15.0
    ref = (torch.from_numpy(codes).to(torch.bfloat16) * scale.unsqueeze(3) + t(mn).unsqueeze(3)).float().numpy()
    assert np.array_equal(kh, ref)
    assert np.max(np.abs(kh - k.reshape(kh.shape))) <= np.max(kivi.kivi_scale(mn, mx)) * 0.51 + 1e-2


def test_format_q_k_codes_equal_format_r_with_group_32(rng):
    k = gaussian_bf16(rng, (2, 2, 96, 128), outlier_channels=4)
    v = gaussian_bf16(rng, (2, 2, 96, 128))
    q = kivi.quantize_kivi4(k, v)
    _, _, _, packed_r = kivi.encode_chunks_ref(k, 32)
    assert np.array_equal(kivi.k_words_from_lane_order(q.k_codes), packed_r)


def test_lane_order_relayouts_are_the_documented_bijections(rng):
    w = rng.integers(0, 2 ** 31, size=(3, 16, 32)).astype(np.int32)
    lo = kivi.k_words_to_lane_order(w)
    assert np.array_equal(kivi.k_words_from_lane_order(lo), w)
    vc = rng.integers(0, 16, size=(3, 32, 128)).astype(np.uint8)
    vw = kivi.v_codes_to_words(vc)
    assert np.array_equal(kivi.v_words_to_codes(vw), vc)
    assert np.array_equal(kivi.v_codes_to_words(kivi.v_words_to_codes(
        rng.integers(-2 ** 31, 2 ** 31, size=(2, 512)).astype(np.int32))).shape, (2, 512))
    for m in range(2):
        for g in range(4):
            for c in range(16):
                for s in range(4):
                    assert lo[1, m * 256 + (16 * g + c) * 4 + s] == w[1, 4 * s + g, 16 * m + c]
    # V: lane 16g + c's word P of half m holds channels 32P + 2c, 32P + 2c + 1
    # (one 32-channel scale group) and only tokens 16m + 4g .. 16m + 4g + 3
    for m in range(2):
        for g in range(4):
            for c in range(16):
                for P in range(4):
                    w = int(vw[2, m * 256 + (16 * g + c) * 4 + P]) & 0xFFFFFFFF
                    got = sorted(((w >> (4 * n)) & 15) for n in range(8))
                    want = sorted(int(x) for x in vc[2, 16 * m + 4 * g:16 * m + 4 * g + 4,
                                                     32 * P + 2 * c:32 * P + 2 * c + 2].reshape(-1))
                    assert got == want


def test_format_q_pages_are_separate_blocks(rng):
    """A 16-token page (half of a 32-token group) owns K code words m*256..,
    V code words m*256.. and V metadata block m; changing the other half's
    tokens leaves them untouched (only the per-channel K metadata is shared)."""
    k = gaussian_bf16(rng, (1, 2, 64, 128), outlier_channels=2)
    v = gaussian_bf16(rng, (1, 2, 64, 128))
    a = kivi.quantize_kivi4(k, v)
    for m in range(2):
        k2, v2 = k.copy(), v.copy()
        other = slice(16 * (1 - m), 16 * (1 - m) + 16)
        for t in (other, slice(32 + 16 * (1 - m), 32 + 16 * (1 - m) + 16)):
            v2[:, :, t] = gaussian_bf16(rng, v2[:, :, t].shape)
            k2[:, :, t] = np.clip(gaussian_bf16(rng, k2[:, :, t].shape), k.min(), k.max())
        b = kivi.quantize_kivi4(k2, v2)
        own = slice(256 * m, 256 * m + 256)
        assert np.array_equal(a.v_codes[..., own], b.v_codes[..., own])
        assert np.array_equal(a.v_meta[..., m, :, :, :, :], b.v_meta[..., m, :, :, :, :])
        assert not np.array_equal(a.v_codes[..., 256 * (1 - m):256 * (1 - m) + 256],
                                  b.v_codes[..., 256 * (1 - m):256 * (1 - m) + 256])


def test_format_q_metadata_and_codes_consistent(rng):
    k = gaussian_bf16(rng, (1, 3, 64, 128), outlier_channels=2)
    v = gaussian_bf16(rng, (1, 3, 64, 128), outlier_channels=2)
    c = kivi.quantize_kivi4(k, v)
    kc, ks, kz, vc, vs, vz = kivi.kivi4_codes_and_meta(k, v)
    kh, vh = kivi.dequant_kivi4(c)
    kh2 = (kc.reshape(1, 3, 2, 32, 128) * ks[:, :, :, None].astype(np.float64)
           + kz[:, :, :, None]).reshape(kh.shape)
    vh2 = vc * np.repeat(vs, 32, -1).astype(np.float64) + np.repeat(vz, 32, -1)
    assert np.array_equal(kh, kh2) and np.array_equal(vh, vh2)
    # zero == group minimum exactly (fp16 holds these bf16 values)
    assert np.array_equal(kz, k.reshape(1, 3, 2, 32, 128).min(axis=3))
    # reconstruction error: half a step plus the bf16 roundings of the ladder
    assert np.all(np.abs(kh - k) <= np.repeat(ks, 32, axis=2) * 0.65 + 1e-3)
    # every slot of k_meta points at the channel KSLOT says
    for p in range(16):
        for s in range(8):
            ch = 8 * p + kivi.KSLOT[s]
            assert np.array_equal(c.k_meta[..., p, 0, s], f16_bits(kivi.kivi_scale(
                k.reshape(1, 3, 2, 32, 128).min(axis=3), k.reshape(1, 3, 2, 32, 128).max(axis=3))[..., ch]))


def test_attention_oracle_textbook_and_lse_split(rng):
    bs, hq, hkv, n = 2, 8, 2, 70
    q = gaussian_bf16(rng, (bs, hq, 128))
    k = rng.standard_normal((bs, hkv, n, 128))
    v = rng.standard_normal((bs, hkv, n, 128))
    sc = 1 / np.sqrt(128)
    out, lse = kivi.attention(q, k, v, sc, return_lse=True)
    # explicit loops for one head
    b, h = 1, 5
    s = np.array([np.dot(q[b, h].astype(np.float64), k[b, h // 4, t]) for t in range(n)]) * sc
    w = np.exp(s - s.max())
    ref = (w[:, None] * v[b, h // 4]).sum(0) / w.sum()
    assert np.allclose(out[b, h], ref, atol=1e-12)
    # split at an arbitrary point and LSE-merge (lse_merge.py:79-119)
    o1, l1 = kivi.attention(q, k[:, :, :23], v[:, :, :23], sc, return_lse=True)
    o2, l2 = kivi.attention(q, k[:, :, 23:], v[:, :, 23:], sc, return_lse=True)
    m = np.maximum(l1, l2)
    w1, w2 = np.exp(l1 - m)[..., None], np.exp(l2 - m)[..., None]
    assert np.allclose((w1 * o1 + w2 * o2) / (w1 + w2), out, atol=1e-12)


def test_lse_merge_of_two_segments_is_attention_over_both(rng):
    """Closed form: merging the normalised outputs of two KV segments by their
    LSEs equals attention over the concatenated segments."""
    q = gaussian_bf16(rng, (2, 8, 128))
    k = gaussian_bf16(rng, (2, 2, 70, 128))
    v = gaussian_bf16(rng, (2, 2, 70, 128))
    sc = 1 / np.sqrt(128)
    oa, la = okivi.attention(q, k[:, :, :23], v[:, :, :23], sc, return_lse=True)
    ob, lb = okivi.attention(q, k[:, :, 23:], v[:, :, 23:], sc, return_lse=True)
    full = okivi.attention(q, k, v, sc)
    assert np.allclose(okivi.lse_merge(oa, la, ob, lb), full, atol=1e-12)
    # the LSE itself: log of the softmax denominator
    s = np.einsum("bhgd,bhnd->bhgn", q.reshape(2, 2, 4, 128).astype(np.float64), k.astype(np.float64)) * sc
    _, lfull = okivi.attention(q, k, v, sc, return_lse=True)
    assert np.allclose(lfull, np.log(np.exp(s).sum(-1)).reshape(2, 8), atol=1e-10)


def test_torch_cpu_restatement_equals_oracle_attention(rng):
    """The torch-CPU C2 step (bench.py's CPU baseline) against the numpy
    oracle's dequant + float64 attention on the same Format Q cache."""
    import torch
    from oracle import torch_cpu
    B, KV, HQ, G, R = 2, 2, 8, 3, 40
    k = gaussian_bf16(rng, (B, KV, G * 32, 128), outlier_channels=2)
    v = gaussian_bf16(rng, (B, KV, G * 32, 128))
    c = kivi.quantize_kivi4(k, v)
    kr = gaussian_bf16(rng, (B, KV, R, 128))
    vr = gaussian_bf16(rng, (B, KV, R, 128))
    q = gaussian_bf16(rng, (B, HQ, 128))
    ref = kivi.kivi4_decode_attention(q, c, G, kr, vr, R, 1 / np.sqrt(128))
    prep = torch_cpu.prepare_c2(c.k_codes, c.k_meta, c.v_codes, c.v_meta, kr, vr)
    got = torch_cpu.decode_attention(torch.from_numpy(q.astype(np.float32)), prep, 1 / np.sqrt(128)).numpy()
    assert got.shape == ref.shape and np.abs(got - ref).max() <= 1e-5


def test_torch_cpu_c3_step_equals_oracle(rng):
    """The torch-CPU C3 step (bench.py's C3 CPU baseline): Quest bounds within
    fp32 summation-order rounding of the oracle's, the same top pages where
    the bounds are separated, and the sparse attention over those pages equal
    to the oracle's dequant + attention."""
    import torch
    from oracle import select as osel
    from oracle import torch_cpu
    B, KV, HQ, G, n_sel = 2, 2, 8, 8, 5
    k = gaussian_bf16(rng, (B, KV, G * 32, 128), outlier_channels=2)
    v = gaussian_bf16(rng, (B, KV, G * 32, 128))
    q = gaussian_bf16(rng, (B, HQ, 128))
    c = kivi.quantize_kivi4(k, v)
    pmin, pmax = osel.page_minmax_f16(k)
    raw_q = osel.gqa_mean_query(q, KV)
    prep = torch_cpu.prepare_c3(raw_q, pmin, pmax, c.k_codes, c.k_meta, c.v_codes, c.v_meta)
    from oracle.numerics import f16_to_f32
    ref_sc = osel.quest_chunk_score(raw_q, f16_to_f32(pmin), f16_to_f32(pmax), 2 * G)
    got_sc = torch_cpu.quest_scores(prep).numpy()
    assert np.abs(got_sc - ref_sc).max() <= 1e-4 * np.abs(ref_sc).max()
    sel, out = torch_cpu.c3_step(torch.from_numpy(q.astype(np.float32)), prep, n_sel, 1 / np.sqrt(128))
    ref_sel = osel.topk_indices(ref_sc, n_sel)
    s = np.sort(ref_sc, axis=-1)[..., ::-1]
    if (s[..., n_sel - 1] - s[..., n_sel] > 1e-3 * np.abs(s).max()).all():
        assert np.array_equal(sel.numpy(), np.sort(ref_sel, axis=-1))
    z = np.zeros((B, KV, 0, 128), np.float32)
    ref = kivi.kivi4_sparse_attention(q, c, G, z, z, 0, sel.numpy(), 1 / np.sqrt(128))
    assert np.abs(out.numpy() - ref).max() <= 1e-5


def test_torch_cpu_c4_search_equals_oracle():
    """The torch-CPU C4 search (bench.py's C4 CPU baseline) against the numpy
    oracle: the query codes, the candidate sets and the exact scores."""
    import torch
    from oracle import rabitq as orq
    from oracle import torch_cpu
    from oracle.numerics import f16_to_f32
    rng = np.random.default_rng(5)
    keys = orq.clustered_unit_keys(rng, 4096, 16)
    qs = orq.clustered_unit_keys(rng, 12, 16)
    signs = orq.srht_signs(42)
    codes, fac = orq.encode(keys, signs)
    cand_ref, _, _ = orq.search(qs, keys, codes, fac, signs, 64)
    prep = torch_cpu.prepare_c4(keys, codes, fac, signs)
    cand, exact = torch_cpu.c4_search(torch.from_numpy(f16_to_f32(qs)), prep, 64, q_block=5)
    # the popcount path itself: query codes equal the oracle's encode
    y = (torch.from_numpy(f16_to_f32(qs)) * prep["signs"]) @ prep["H"]
    bits = (y >= 0).to(torch.int64).view(-1, 16, 8)
    cq = (bits << torch.arange(8)).sum(-1).to(torch.uint8).numpy()
    assert np.array_equal(cq, orq.encode(qs, signs)[0])
    overlap = np.mean([len(set(a) & set(b)) / 64 for a, b in zip(cand.numpy(), cand_ref)])
    assert overlap >= 0.98
    ref_exact = orq.exact_scores(qs, keys, cand.numpy())
    assert np.abs(exact.numpy() - ref_exact).max() <= 1e-5
    # the 64-bit SWAR bit count against a byte table
    w = torch.from_numpy(rng.integers(-2**63, 2**63 - 1, size=1000, dtype=np.int64))
    table = np.array([bin(i).count("1") for i in range(256)])
    ref_pc = table[w.numpy().view(np.uint8).reshape(-1, 8)].sum(-1)
    assert np.array_equal(torch_cpu._popc64(w).numpy(), ref_pc)


def test_token_attention_oracle_reduces_to_pages_and_dense(rng):
    """The token-list oracle pinned by the two attention oracles it
    generalises: listing every token of some 16-token pages (in any order,
    with bf16 tail rows mapped in) equals the page-sparse oracle over those
    pages with the same rows as its residual window; listing every quantized
    token plus the tail equals dense attention over the cache + residual;
    a repeated token equals attending its duplicated row; ids outside both
    zones are skipped."""
    bs, hq, kv, ng, n_tail = 1, 8, 2, 6, 5
    k = gaussian_bf16(rng, (bs, kv, ng * 32, 128), outlier_channels=1)
    v = gaussian_bf16(rng, (bs, kv, ng * 32, 128))
    rec = okivi.quantize_kivi4(k, v)
    rows_k = gaussian_bf16(rng, (bs, kv, 40, 128))
    rows_v = gaussian_bf16(rng, (bs, kv, 40, 128))
    q = gaussian_bf16(rng, (bs, hq, 128))
    sc = 1 / np.sqrt(128)
    tail0, near0, near_len = 3, 10, 20
    q_end = 32 * ng
    # pages 2, 5, 9, their tokens shuffled, plus two tail tokens; the near rows
    pages = np.array([[[2, 5, 9]] * kv])
    toks = (pages[..., None] * 16 + np.arange(16)).reshape(bs, kv, -1)
    toks = np.stack([[rng.permutation(toks[0, h]) for h in range(kv)]])
    tl = np.concatenate([toks, np.full((bs, kv, 1), q_end + 1), np.full((bs, kv, 1), q_end + 4)], -1)
    got, lse = okivi.kivi4_token_attention(q, rec, ng, rows_k, rows_v, tl, tail0, n_tail, near0, near_len, sc,
                                           return_lse=True)
    res_k = np.concatenate([rows_k[:, :, [tail0 + 1, tail0 + 4]], rows_k[:, :, near0:near0 + near_len]], 2)
    res_v = np.concatenate([rows_v[:, :, [tail0 + 1, tail0 + 4]], rows_v[:, :, near0:near0 + near_len]], 2)
    want, wlse = okivi.kivi4_sparse_attention(q, rec, ng, res_k, res_v, res_k.shape[2], pages, sc, return_lse=True)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12) and np.allclose(lse, wlse, rtol=1e-12)
    # every quantized token + the whole tail = dense attention
    every = np.broadcast_to(np.arange(q_end + n_tail), (bs, kv, q_end + n_tail))
    got = okivi.kivi4_token_attention(q, rec, ng, rows_k, rows_v, every, tail0, n_tail, near0, 0, sc)
    dense = okivi.kivi4_decode_attention(q, rec, ng, rows_k[:, :, tail0:tail0 + n_tail],
                                         rows_v[:, :, tail0:tail0 + n_tail], n_tail, sc)
    assert np.allclose(got, dense, rtol=1e-12, atol=1e-12)
    # a repeated token and skipped ids (negative, past the tail)
    tl2 = np.array([[[7, 7, -1, q_end + n_tail, 40]] * kv])
    got = okivi.kivi4_token_attention(q, rec, ng, rows_k, rows_v, tl2, tail0, n_tail, near0, 0, sc)
    kh, vh = okivi.dequant_kivi4(rec)
    want = okivi.attention(q, kh[:, :, [7, 7, 40]], vh[:, :, [7, 7, 40]], sc)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
