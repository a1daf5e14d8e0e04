"""Pins of the Quest / top-k / density / stage-2 / RaBitQ oracles (CPU)."""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import rabitq, select
from oracle.kivi import encode_chunks_ref
from oracle.numerics import bf16r, f16_bits, f16_to_f32
from tests.helpers import gaussian_bf16


# ------------------------------- Quest ------------------------------------
def test_quest_score_is_an_upper_bound_and_handles_invalid(rng):
    k = gaussian_bf16(rng, (2, 3, 20 * 16, 128), outlier_channels=4)
    q = gaussian_bf16(rng, (2, 3, 128))
    mn, mx, _, _ = encode_chunks_ref(k, 16)
    valid = np.ones((2, 3, 20), dtype=bool)
    valid[1, 2, 7] = False
    s = select.quest_chunk_score(q, mn, mx, 18, valid)
    assert s.shape == (2, 3, 18) and s.dtype == np.float32
    assert np.isneginf(s[1, 2, 7]) and np.isfinite(s).sum() == s.size - 1
    ok = valid[:, :, :18]
    kc = k.reshape(2, 3, 20, 16, 128)[:, :, :18]
    assert select.quest_upper_bound_holds(q, kc, np.where(ok, s, np.inf))
    # float64 reference sum: the canonical order differs only by fp32 rounding
    ref = np.maximum(q[:, :, None].astype(np.float64) * mn[:, :, :18], q[:, :, None] * mx[:, :, :18]).sum(-1)
    assert np.allclose(s[ok], ref[ok], rtol=1e-5, atol=1e-4)


def test_quest_score_exact_on_dyadic_inputs(rng):
    # small integers: every partial sum is exact, so any order gives the same bits
    q = rng.integers(-8, 8, size=(1, 2, 128)).astype(np.float32)
    mn = rng.integers(-8, 8, size=(1, 2, 5, 128)).astype(np.float32)
    mx = mn + rng.integers(0, 8, size=mn.shape).astype(np.float32)
    s = select.quest_chunk_score(q, mn, mx, 5)
    ref = np.maximum(q[:, :, None] * mn, q[:, :, None] * mx).sum(-1)
    assert np.array_equal(s, ref.astype(np.float32))


def test_quest_products_match_torch_fp32(rng):
    q = gaussian_bf16(rng, (1, 1, 128))
    mn = gaussian_bf16(rng, (1, 1, 4, 128))
    prod = torch.from_numpy(q).unsqueeze(2) * torch.from_numpy(mn)
    exact = q[:, :, None].astype(np.float64) * mn
    assert np.array_equal(prod.numpy().astype(np.float64), exact)     # bf16*bf16 exact in fp32


# ------------------------------- top-k ------------------------------------
def test_topk_matches_argsort_on_tie_free_inputs(rng):
    x = rng.permutation(5000).astype(np.float32).reshape(2, 2500) - 1234.5
    sel = select.topk_indices(x, 100)
    for r in range(2):
        assert set(sel[r]) == set(np.argsort(-x[r])[:100])
        assert np.all(np.diff(sel[r]) > 0)


def test_topk_ties_and_sentinel():
    x = np.array([[1.0, 3.0, 3.0, 3.0, 0.5, 3.0]], dtype=np.float32)
    assert select.topk_indices(x, 3).tolist() == [[1, 2, 3]]
    assert select.topk_indices(np.array([[2.0, 1.0]], np.float32), 4).tolist() == [[0, 1, -1, -1]]
    # -inf / huge negatives rank last, +inf first
    y = np.array([[-np.inf, 5.0, np.inf, -1e30, 0.0]], dtype=np.float32)
    assert select.topk_indices(y, 2).tolist() == [[1, 2]]


def test_topk_gather_concat_layout(rng):
    sc = rng.permutation(64).astype(np.float32).reshape(1, 1, 64)
    lut = (np.arange(64) * 7 + 3).reshape(1, 1, 64)
    skipped = np.array([[[900, 901, 902]]])
    out = select.topk_gather_concat(sc, lut, skipped, 5, 10)
    top = np.argsort(-sc[0, 0])[:5]
    assert set(out[0, 0, :5]) == set(lut[0, 0, top]) and out[0, 0, 5:8].tolist() == [900, 901, 902]
    assert out[0, 0, 8:].tolist() == [0, 0]


# ------------------------------- density ----------------------------------
def test_density_tree_sum(rng):
    cent = gaussian_bf16(rng, (1, 2, 10, 128))
    q = gaussian_bf16(rng, (1, 2, 128))
    ids = np.array([[[3, 0, 9, -1, 10], [1, 1, 2, 3, 4]]])
    s = select.chunk_density_scores(ids, cent, q)
    for h in range(2):
        for j in range(5):
            i = ids[0, h, j]
            if 0 <= i < 10:
                ref = math.fsum(float(a) * float(b) for a, b in zip(cent[0, h, i], q[0, h]))
                assert abs(s[0, h, j] - ref) <= 1e-5 * (1 + abs(ref))
            else:
                assert s[0, h, j] == np.float32(-1e30)
    qi = np.arange(128, dtype=np.float32)[None, None] % 7
    ci = (np.arange(128, dtype=np.float32) % 5)[None, None, None].repeat(2, axis=2)
    assert select.chunk_density_scores(np.array([[[1]]]), ci, qi)[0, 0, 0] == np.float32((qi * ci[:, :, 0]).sum())


def test_dense_mask():
    pos = np.array([[[0, 3, 7, 12]]])
    m = select.dense_mask_from_topk(pos, 8)
    assert m.tolist() == [[[True, False, False, True, False, False, False, True]]]


# ------------------------------- stage-2 ----------------------------------
def test_bitonic_network_sorts_descending(rng):
    for n in (8, 16):
        s = rng.permutation(1000).astype(np.float32)[: 5 * n].reshape(5, n)
        t = np.arange(5 * n).reshape(5, n)
        ss, tt = select.bitonic_desc(s, t)
        assert np.array_equal(ss, -np.sort(-s, axis=-1))
        for r in range(5):                  # indices travel with their scores
            assert np.array_equal(s[r][tt[r] - r * n], ss[r])


def test_stage2_products_match_torch_bf16_ops(rng):
    """Per-dim bf16 products of the oracle equal torch's bf16 ops on the same
    dequantized keys (qk_dot.py:101-145 with the chunk's scale / min)."""
    g = 16
    k = gaussian_bf16(rng, (1, 2, 6 * g, 128), outlier_channels=2)
    q = gaussian_bf16(rng, (1, 2, 128))
    mn, mx, _, packed = encode_chunks_ref(k, g)
    ids = np.array([[[4, 1, 0], [2, 5, 3]]])
    dm = np.array([[[True, False, False], [False, True, False]]])
    sc, ix = select.kivi_qk_dense_sparse(ids, dm, packed, mn, mx, q, 16, 8, g)
    # torch restatement of the dequant + product with bf16 tensors
    from oracle.kivi import unpack_last_dim
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)
    codes = unpack_last_dim(np.swapaxes(packed, -1, -2))
    for h in range(2):
        for j, c in enumerate(ids[0, h]):
            scale = (t(mx[0, h, c]) - t(mn[0, h, c])) / 15.0
            kh = torch.from_numpy(codes[0, h, c]).to(torch.bfloat16) * scale + t(mn[0, h, c])
            p = (kh * t(q[0, h])).float().numpy()                       # [g, 128]
            acc = np.zeros(g, np.float32)
            for d in range(128):
                acc = (acc + p[:, d]).astype(np.float32)
            order = np.argsort(-acc, kind="stable")
            kk = 16 if dm[0, h, j] else 8
            got = sc[0, h, j * g:(j + 1) * g]
            assert np.array_equal(got[:kk], acc[order][:kk])
            assert np.all(got[kk:] == np.float32(-1e30))
            assert set(ix[0, h, j * g:j * g + kk]) == set(c * g + order[:kk])


def test_gqa_mean_matches_torch(rng):
    q = gaussian_bf16(rng, (2, 32, 128))
    ref = torch.from_numpy(q).to(torch.bfloat16).view(2, 8, 4, 128).mean(dim=2).float().numpy()
    assert np.array_equal(select.gqa_mean_query(q, 8), ref)


# ------------------------------- RaBitQ -----------------------------------
def test_fwht_is_the_sylvester_hadamard_matrix(rng):
    x = rng.standard_normal((3, 128)).astype(np.float32)
    H = scipy.linalg.hadamard(128).astype(np.float64)
    assert np.allclose(rabitq.fwht(x), x.astype(np.float64) @ H.T, atol=1e-4)


def test_popcount_identity_brute_force(rng):
    keys = f16_bits(rng.standard_normal((40, 128)).astype(np.float32))
    qs = f16_bits(rng.standard_normal((5, 128)).astype(np.float32))
    sg = rabitq.srht_signs(7)
    ck, _ = rabitq.encode(keys, sg)
    cq, _ = rabitq.encode(qs, sg)
    sk = np.where(rabitq.fwht(f16_to_f32(keys) * sg) >= 0, 1, -1)
    sq = np.where(rabitq.fwht(f16_to_f32(qs) * sg) >= 0, 1, -1)
    assert np.array_equal(128 - 2 * rabitq.popcount_distance(cq, ck), sq @ sk.T)
    # bit b of byte j is dim 8j + b
    bits = np.unpackbits(ck, axis=-1, bitorder="little")
    assert np.array_equal(bits, (sk > 0).astype(np.uint8))


def test_correction_factor_closed_form(rng):
    x = rng.standard_normal((20, 128)).astype(np.float32)
    _, fac = rabitq.encode(f16_bits(x), rabitq.srht_signs(3))
    xx = f16_to_f32(f16_bits(x)).astype(np.float64)
    y = xx * rabitq.srht_signs(3) @ scipy.linalg.hadamard(128).T
    o = y / np.linalg.norm(y, axis=1, keepdims=True)
    inv = 1.0 / (np.abs(o).sum(1) / np.sqrt(128))
    assert np.allclose(f16_to_f32(fac[:, 1]), inv, rtol=2e-3)
    assert np.allclose(f16_to_f32(fac[:, 0]), np.linalg.norm(xx, axis=1), rtol=1e-3)


def _vectors_with_srht_images(y: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """fp16 vectors x whose SRHT image H (signs * x) is y (up to the fp16
    rounding of x): H H = 128 I for the Sylvester matrix, so x = signs * H y / 128."""
    H = scipy.linalg.hadamard(128).astype(np.float64)
    return f16_bits(((y @ H.T) / 128.0 * signs).astype(np.float32))


def test_estimate_closed_form_on_hand_built_srht_images():
    """est(q, k) = ||k|| ||q|| / (alpha_k alpha_q) <sign y_k, sign y_q> / 128,
    alpha = <sign(y) / sqrt(128), y / ||y||> (the RaBitQ alignment <o_bar, o>,
    PC:1181-1193 "weight = (r / alpha) ||k||"), computed in float64 from the
    fp16 inputs.  The images are built by hand with sum|y| far from
    ||y|| sqrt(128) (alpha 0.4 .. 0.9), so dropping or inverting either
    correction moves the estimate by 10% or more, far outside the fp16
    rounding of the stored factors."""
    D = 128
    sg = rabitq.srht_signs(5)
    g = np.random.default_rng(9)
    mags = [np.r_[np.full(8, 20.0), np.ones(120)],          # alpha ~ 0.43
            np.r_[np.ones(64), np.full(64, 5.0)],            # alpha ~ 0.83
            1.0 + np.arange(D) % 7,                           # alpha ~ 0.91
            np.r_[np.full(32, 9.0), np.full(96, 1.5)],        # alpha ~ 0.68
            np.geomspace(1.0, 40.0, D)]                       # alpha ~ 0.7
    def build(n, scale):
        y = np.stack([mags[i % len(mags)] * g.choice([-1.0, 1.0], size=D) for i in range(n)])
        return _vectors_with_srht_images(y * scale[:, None], sg)
    keys = build(12, g.uniform(0.05, 3.0, size=12))
    qs = build(5, g.uniform(0.05, 3.0, size=5))
    ck, fk = rabitq.encode(keys, sg)
    cq, fq = rabitq.encode(qs, sg)
    est = rabitq.estimate(cq, fq, ck, fk).astype(np.float64)

    H = scipy.linalg.hadamard(D).astype(np.float64)
    def parts(x16):
        x = f16_to_f32(x16).astype(np.float64)
        y = (x * sg) @ H.T
        s = np.where(y >= 0, 1.0, -1.0)
        alpha = (s / np.sqrt(D) * (y / np.linalg.norm(y, axis=1, keepdims=True))).sum(1)
        return np.linalg.norm(x, axis=1), alpha, s
    nk, ak, sk = parts(keys)
    nq, aq, sq = parts(qs)
    assert np.all(ak < 0.92) and np.all(aq < 0.92) and ak.min() < 0.5
    dots = sq @ sk.T / D
    expected = nq[:, None] * nk[None, :] / (aq[:, None] * ak[None, :]) * dots
    tol = 4e-3 * np.abs(expected) + 1e-9
    assert np.all(np.abs(est - expected) <= tol)
    # the same check rejects the plausible mistakes (self-test of its power)
    for wrong in (expected * ak[None, :], expected * aq[:, None],                 # a correction dropped
                  expected * ak[None, :] ** 2, expected * aq[:, None] ** 2,       # a correction inverted
                  nq[:, None] * nk[None, :] * dots):                             # both dropped
        assert not np.all(np.abs(est - wrong) <= 4e-3 * np.abs(wrong) + 1e-9)


def test_estimate_tracks_inner_product_and_exact_rerank(rng):
    keys = rabitq.clustered_unit_keys(rng, 4096, 16)
    qs = rabitq.clustered_unit_keys(rng, 4, 16)
    sg = rabitq.srht_signs(42)
    ck, fk = rabitq.encode(keys, sg)
    cq, fq = rabitq.encode(qs, sg)
    est = rabitq.estimate(cq, fq, ck, fk)
    exact = f16_to_f32(qs).astype(np.float64) @ f16_to_f32(keys).astype(np.float64).T
    # 1-bit x 1-bit is a coarse estimator: clearly correlated, far from random
    for i in range(4):
        assert np.corrcoef(est[i], exact[i])[0, 1] > 0.5
    cand, fi, fs = rabitq.search(qs, keys, ck, fk, sg, 256)
    ex = rabitq.exact_scores(qs, keys, fi)
    assert np.array_equal(ex, fs) and np.all(np.diff(fs, axis=-1) <= 0)
    assert np.allclose(fs, np.take_along_axis(exact, fi, -1), atol=1e-5)
    # recall of the true top-16 inside the 256 estimated candidates (random: 6%)
    true16 = np.argsort(-exact, axis=-1)[:, :16]
    rec = np.mean([len(set(true16[i]) & set(cand[i])) / 16 for i in range(4)])
    assert rec >= 0.4


# --------------------------- fp16 page metadata ----------------------------
def test_f16_directed_rounding_is_tight_over_all_bf16():
    from oracle.numerics import bf16_to_f32
    x = bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    fin = np.isfinite(x)
    x = x[fin]
    dn = select.f16_directed(x, False).view(np.float16)
    up = select.f16_directed(x, True).view(np.float16)
    with np.errstate(over="ignore"):
        assert np.all(dn.astype(np.float32) <= x) and np.all(up.astype(np.float32) >= x)
        # tight: the next fp16 past each bound crosses x
        nxt = np.nextafter(dn, np.float16(np.inf)).astype(np.float32)
        prv = np.nextafter(up, np.float16(-np.inf)).astype(np.float32)
    assert np.all(nxt[np.isfinite(dn)] > x[np.isfinite(dn)])
    assert np.all(prv[np.isfinite(up)] < x[np.isfinite(up)])
    # bf16 values inside fp16's normal range convert exactly
    ok = (np.abs(x) >= 2.0 ** -14) & (np.abs(x) <= 65504)
    assert np.array_equal(dn[ok].astype(np.float32), x[ok]) and np.array_equal(up[ok].astype(np.float32), x[ok])


def test_page_minmax_brute_force(rng):
    k = gaussian_bf16(rng, (1, 2, 48, 128))
    k[0, 1, 5, 7] = 1e6                              # beyond fp16: max rounds up to +inf
    k[0, 0, 20, 3] = -3e-9                           # below fp16 subnormals: min rounds down
    mn, mx = select.page_minmax_f16(k, 16)
    for h in range(2):
        for p in range(3):
            for d in (0, 3, 7, 127):
                col = k[0, h, 16 * p:16 * p + 16, d]
                lo, hi = np.float16(mn[0, h, p, d].view(np.float16)), np.float16(mx[0, h, p, d].view(np.float16))
                assert float(lo) <= col.min() and float(hi) >= col.max()
    assert np.isposinf(mx[0, 1, 0, 7].view(np.float16))
    assert mn[0, 0, 1, 3].view(np.float16) < 0


# --------------------------- sparse attention ------------------------------
def test_sparse_attention_oracle_invariants(rng):
    from oracle import kivi as okivi
    bs, kv, hq, ng, res = 1, 2, 8, 6, 20
    k = gaussian_bf16(rng, (bs, kv, ng * 32, 128), outlier_channels=2)
    v = gaussian_bf16(rng, (bs, kv, ng * 32, 128))
    cache = okivi.quantize_kivi4(k, v)
    kr = gaussian_bf16(rng, (bs, kv, res, 128))
    vr = gaussian_bf16(rng, (bs, kv, res, 128))
    q = gaussian_bf16(rng, (bs, hq, 128))
    sc = 1 / np.sqrt(128)
    all_pages = np.broadcast_to(np.arange(2 * ng), (bs, kv, 2 * ng))
    dense = okivi.kivi4_decode_attention(q, cache, ng, kr, vr, res, sc)
    assert np.allclose(okivi.kivi4_sparse_attention(q, cache, ng, kr, vr, res, all_pages, sc), dense,
                       atol=1e-12)
    sub = np.array([[[0, 3, 4, 9], [11, 2, 5, 6]]])
    a = okivi.kivi4_sparse_attention(q, cache, ng, kr, vr, res, sub, sc)
    # order and out-of-range ids do not matter; without a residual window,
    # listing every page twice does not either (all weights double)
    b = okivi.kivi4_sparse_attention(q, cache, ng, kr, vr, res, sub[..., ::-1], sc)
    assert np.allclose(a, b, atol=1e-12)
    a0 = okivi.kivi4_sparse_attention(q, cache, ng, kr, vr, 0, sub, sc)
    c0 = okivi.kivi4_sparse_attention(q, cache, ng, kr, vr, 0, np.concatenate([sub, sub, -sub - 1, sub + 99], -1), sc)
    assert np.allclose(a0, c0, atol=1e-12)
    # a single page equals dense attention over a cache truncated to that page
    one = okivi.kivi4_sparse_attention(q, cache, ng, kr, vr, 0, np.zeros((1, 2, 1), int), sc)
    kh, vh = okivi.dequant_kivi4(cache)
    ref = okivi.attention(q, kh[:, :, :16], vh[:, :, :16], sc)
    assert np.allclose(one, ref, atol=1e-12)
