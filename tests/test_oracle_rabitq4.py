"""The 4-bit RaBitQ oracle (oracle/rabitq4.py) against the reference's own
ParisKV code (golden vectors from tests/golden/make_golden_rabitq4.py) and
against closed forms that do not depend on that code."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import scipy.linalg

from oracle import rabitq4 as r4
from oracle.numerics import bf16_bits, bf16_to_f32, bf16r

GOLDEN = Path(__file__).parent / "golden" / "rabitq4_pariskv.npz"


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


def test_levels_are_the_reference_constants(gold):
    """PC:266-270, read from the reference file by the fixture script."""
    assert np.array_equal(bf16_bits(r4.MAG_THRESHOLDS), gold["mag_thresholds"])
    assert np.array_equal(bf16_bits(r4.MAG_CENTERS), gold["mag_centers"])


@pytest.mark.parametrize("h", [0, 1])
def test_key_encode_matches_reference_batch_encode(gold, h):
    """Sign bytes, 4-bit codes and block weights of PC:1130-1195, bit-exact,
    including a zero key, a key of 1e-6 entries, a key of +-3000 and a key
    with one all-zero block."""
    signs = bf16_to_f32(gold["signs"])
    code, packed, w = r4.encode_keys(bf16_to_f32(gold["keys"][0, h]), signs)
    assert np.array_equal(code, gold["codebook"][0, h])
    assert np.array_equal(packed, gold["packed_4bit"][0, h])
    assert np.array_equal(bf16_bits(w), gold["block_weight"][0, h])


@pytest.mark.parametrize("h", [0, 1])
def test_query_blocks_match_reference(gold, h):
    signs = bf16_to_f32(gold["signs"])
    qb, qn = r4.encode_query(bf16_to_f32(gold["q"][0, h]), signs)
    assert np.array_equal(bf16_bits(qb), gold["q_blocks"][0, h])
    assert np.array_equal(bf16_bits(qn), gold["q_norm"][0, h, 0])


def test_decode_matches_reference_unpack(gold):
    """rerank._unpack_4bit_codes: sign (+1 for bit 3) and magnitude index."""
    vals = r4.decode_packed(gold["packed_4bit"])
    want = np.where(gold["unpack_sign"] > 0, r4.MAG_CENTERS[gold["unpack_t"]], -r4.MAG_CENTERS[gold["unpack_t"]])
    assert np.array_equal(vals, want)


@pytest.mark.parametrize("h", [0, 1])
def test_rerank_matches_reference_test_model(gold, h):
    """The reference test's sequential-bf16 model of rerank.cu, bit-exact
    (unsorted candidates, a repeated candidate, the zero and tiny keys)."""
    sc = r4.rerank_scores(gold["cand"][0, h], gold["packed_4bit"][0, h], bf16_to_f32(gold["block_weight"][0, h]),
                          bf16_to_f32(gold["q_blocks"][0, h]), bf16_to_f32(gold["q_norm"][0, h, 0]))
    assert np.array_equal(bf16_bits(sc), gold["scores"][0, h])


def _rotate64(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """fp64 SRHT of the unit rows: H (sigma * x / ||x||) / sqrt(128), H the
    Sylvester Hadamard matrix."""
    H = scipy.linalg.hadamard(128).astype(np.float64)
    xu = x.astype(np.float64) / np.linalg.norm(x.astype(np.float64), axis=-1, keepdims=True)
    return (xu * signs) @ H.T / np.sqrt(128.0)


def test_signs_and_buckets_against_fp64_rotation():
    """Sign bit j of block b = sign of the fp64 rotation, and the 3-bit
    magnitude = the number of thresholds below |u| of the fp64 block
    direction, wherever the fp64 value is clear of 0 and of every threshold."""
    rng = np.random.default_rng(11)
    signs = np.where(rng.integers(0, 2, 128) == 1, 1.0, -1.0).astype(np.float32)
    x = bf16r(rng.standard_normal((400, 128)).astype(np.float32))
    code, packed, _ = r4.encode_keys(x, signs)
    y = _rotate64(x, signs).reshape(400, 16, 8)
    u = np.abs(y / np.linalg.norm(y, axis=-1, keepdims=True))
    bits = (code.T[..., None] >> np.arange(8)) & 1                          # [N, 16, 8]
    clear = np.abs(y) > 2e-2
    assert clear.mean() > 0.7
    assert np.array_equal(bits[clear], (y[clear] > 0).astype(np.uint8))
    v = np.stack([packed & 15, packed >> 4], axis=-1).reshape(16, 400, 8).transpose(1, 0, 2)
    assert np.array_equal(v >> 3, bits)                                     # sign bit inside the 4-bit value
    thr = r4.MAG_THRESHOLDS.astype(np.float64)
    away = np.min(np.abs(u[..., None] - thr), axis=-1) > 2e-2
    assert away.mean() > 0.5
    assert np.array_equal((v & 7)[away], (u[..., None] > thr).sum(-1)[away])


def test_block_weights_against_closed_form():
    """weight = (r / alpha) * ||k||, alpha = sum_j c[t_j] |u_j| (PC:1183-1192),
    in fp64 from the oracle's own buckets: within the bf16 roundings."""
    rng = np.random.default_rng(12)
    signs = np.where(rng.integers(0, 2, 128) == 1, 1.0, -1.0).astype(np.float32)
    x = bf16r((rng.standard_normal((300, 128)) * rng.uniform(0.1, 30, (300, 1))).astype(np.float32))
    _, packed, w = r4.encode_keys(x, signs)
    nrm = np.linalg.norm(x.astype(np.float64), axis=-1)
    y = _rotate64(x, signs).reshape(300, 16, 8)
    r = np.linalg.norm(y, axis=-1)
    t = np.stack([packed & 15, packed >> 4], axis=-1).reshape(16, 300, 8).transpose(1, 0, 2) & 7
    alpha = (r4.MAG_CENTERS[t].astype(np.float64) * np.abs(y / r[..., None])).sum(-1)
    want = r / alpha * nrm[:, None]
    assert np.allclose(w.T, want, rtol=2 ** -6)


def test_rerank_one_hot_scores_are_exact():
    """A query with a single 1.0 at (block b, dimension j), weight 1/8 on
    block b (0 elsewhere) and ||q|| = 4 scores +-center[t] / 2 exactly for a
    key whose 4-bit value there is v = sign << 3 | t: pins the nibble order,
    the sign bit, the block of each weight and the q_norm factor."""
    seq = 16
    for b in range(16):
        for j in range(8):
            packed = np.zeros((16, seq, 4), dtype=np.uint8)
            v = np.arange(16, dtype=np.uint8)
            packed[b, :, j // 2] = v << 4 if j % 2 else v
            w = np.zeros((16, seq), dtype=np.float32)
            w[b] = 0.125
            qb = np.zeros((16, 8), dtype=np.float32)
            qb[b, j] = 1.0
            got = r4.rerank_scores(np.arange(seq), packed, w, qb, np.float32(4.0))
            want = np.where(v & 8, r4.MAG_CENTERS[v & 7], -r4.MAG_CENTERS[v & 7]) / 2
            assert np.array_equal(got, want.astype(np.float32)), (b, j)


def test_rerank_out_of_range_candidates_score_minus_inf():
    rng = np.random.default_rng(13)
    packed = rng.integers(0, 256, (16, 10, 4)).astype(np.uint8)
    w = bf16r(rng.uniform(0, 2, (16, 10)).astype(np.float32))
    qb = bf16r(rng.standard_normal((16, 8)).astype(np.float32))
    sc = r4.rerank_scores(np.array([3, -1, 10, 9]), packed, w, qb, np.float32(1.5))
    assert np.isneginf(sc[1]) and np.isneginf(sc[2]) and np.isfinite(sc[[0, 3]]).all()
    assert sc[0] == r4.rerank_scores(np.array([3]), packed, w, qb, np.float32(1.5))[0]


def test_topk_is_the_k_largest_in_position_order():
    rng = np.random.default_rng(14)
    scores = bf16r(rng.standard_normal(500).astype(np.float32)).round(1)   # many ties
    cand = rng.permutation(10000)[:500]
    got = r4.topk_gather(scores, cand, 37)
    pos = sorted(range(500), key=lambda i: (-float(scores[i]), i))[:37]
    assert np.array_equal(got, cand[np.sort(pos)])
