"""The oracle against golden vectors written by the reference's own
pure-PyTorch functions (tests/golden/make_golden.py):

* KIVI quantise / pack / dequant (Z/cache_hub/kivi/quant_pack.py:86-198) and
  the chunk statistics + chunk-major relayout (S:2133-2135, S:2017): bit-exact.
* The stage-2 scorer (Z/cache_hub/kivi/qk_dot.py:114-175).  The torch
  reference sums the bf16 products in a bf16 tensor (fp32 accumulation, one
  bf16 rounding of the total); the oracle follows the CUDA kernel's
  sequential fp32 sum (kivi_qk_dot.cu:236-284).  So bf16(oracle) equals the
  fixture, or sits one bf16 unit away where the two sums straddle a rounding
  boundary, and the kept token sets agree wherever the boundary scores differ.
* Quest (Z/cache_hub/quest/quest_ops.py:22-31): the torch path rounds each
  product to bf16 before the max and the sum; the CUDA order the oracle
  follows keeps exact fp32 products.  The gap is bounded by the product
  roundings plus the final bf16 rounding.
* lse_merge_torch (Z/cache_hub/lse_merge/lse_merge.py:79-119): fp32 result
  within fp32 rounding of the float64 oracle; bf16 within one bf16 unit.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import kivi as okivi
from oracle import select as osel
from oracle.numerics import bf16_to_f32, bf16r

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLDEN / f"{name}.npz")


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |x| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), np.float32(2.0 ** -126))))
    return np.float32(2.0) ** (e - 7)


@pytest.mark.parametrize("g", [8, 16, 32])
def test_golden_kivi_quant_pack(g):
    f = load("kivi_quant_pack")
    K = bf16_to_f32(f["K"])
    bs, kv, n, d = K.shape
    kc = K.reshape(bs, kv, n // g, g, d)
    mn, mx, mean = okivi.chunk_minmax_mean(kc)
    assert np.array_equal(mn, bf16_to_f32(f[f"g{g}_min"]))
    assert np.array_equal(mx, bf16_to_f32(f[f"g{g}_max"]))
    assert np.array_equal(mean, bf16_to_f32(f[f"g{g}_mean"])), "chunk mean (S:2135)"
    codes = okivi.kivi_codes(kc, mn[..., None, :], mx[..., None, :]).reshape(bs, kv, n, d)
    assert np.array_equal(codes, f[f"g{g}_codes"].astype(np.int32)), "quantize_kcache_4bit codes"
    assert np.array_equal(okivi.kivi_scale(mn, mx), bf16_to_f32(f[f"g{g}_scale"])), "raw scale"
    packed_cm = okivi.pack_chunks_ref(kc, mn, mx)
    assert np.array_equal(packed_cm, f[f"g{g}_packed_cm"]), "chunk-major packed words"
    deq = okivi.dequant_ref(packed_cm, mn, mx).reshape(bs, kv, n, d)
    assert np.array_equal(deq, bf16_to_f32(f[f"g{g}_dequant"])), "unpack_kcache_4bit"


def test_golden_kivi_edge_rows_present():
    """The fixture holds the edge cases it was built for: flat channels (all
    codes 0 through the 1e-8 divisor) and codes 15 at an exact chunk max."""
    f = load("kivi_quant_pack")
    c = f["g32_codes"]
    assert np.all(c[0, 0, :32, :8] == 0)
    assert np.all(c[0, 1, 5, :] == 15) or np.all(f["g8_codes"][0, 1, 5, :] == 15)
    assert c.max() == 15 and c.min() == 0


def stage2_inputs(f, g):
    dense, sparse = (int(x) for x in f[f"g{g}_topk"])
    return dict(chunk_ids=f[f"g{g}_chunk_ids"], dense_mask=f[f"g{g}_dense_mask"],
                packed_K=f[f"g{g}_packed_cm"], chunk_min=bf16_to_f32(f[f"g{g}_min"]),
                chunk_max=bf16_to_f32(f[f"g{g}_max"]), raw_q=bf16_to_f32(f[f"g{g}_raw_q"]),
                dense_topk=dense, sparse_topk=sparse, group_size=g)


def check_stage2_against_golden(s, i, f, g):
    """Scores s / indices i (CUDA-kernel semantics) against the torch fixture."""
    inp = stage2_inputs(f, g)
    ids, mask, dense, sparse = inp["chunk_ids"], inp["dense_mask"], inp["dense_topk"], inp["sparse_topk"]
    ref_s, ref_i = f[f"g{g}_scores"], f[f"g{g}_indices"]
    bs, kv, nk = ids.shape
    s4, i4 = s.reshape(bs, kv, nk, g), i.reshape(bs, kv, nk, g)
    rs4, ri4 = ref_s.reshape(bs, kv, nk, g), ref_i.reshape(bs, kv, nk, g)
    keep = np.where(mask, dense, sparse)
    n_exact = n_kept = n_sets = 0
    for b in range(bs):
        for h in range(kv):
            for c in range(nk):
                k = keep[b, h, c]
                # masked slots: the reference's fill (-3e38, token 0), the CUDA kernel's (-1e30, 0)
                assert np.all(rs4[b, h, c, k:] <= -1e38) and np.all(ri4[b, h, c, k:] == 0)
                assert np.all(s4[b, h, c, k:] == np.float32(-1e30)) and np.all(i4[b, h, c, k:] == 0)
                # every kept score: bf16(ours) within one bf16 unit of the torch value
                ours = dict(zip(i4[b, h, c].tolist(), s4[b, h, c].tolist()))
                for t, rv in zip(ri4[b, h, c, :k].tolist(), rs4[b, h, c, :k].tolist()):
                    if t in ours:
                        ov = bf16r(np.float32(ours[t]))
                        assert abs(ov - rv) <= bf16_ulp(np.float32(rv)), (b, h, c, t, ov, rv)
                        n_exact += int(ov == rv)
                        n_kept += 1
                # the kept sets agree unless the boundary pair is a bf16 near-tie
                full = np.sort(bf16r(s4[b, h, c]))[::-1]
                if k == g or full[k - 1] - full[k] > bf16_ulp(full[k - 1]):
                    assert set(i4[b, h, c, :k].tolist()) == set(ri4[b, h, c, :k].tolist()), (b, h, c)
                    n_sets += 1
    assert n_kept > 0 and n_exact >= 0.9 * n_kept, (n_exact, n_kept)
    assert n_sets >= 0.75 * bs * kv * nk, n_sets


@pytest.mark.parametrize("g", [16, 8])
def test_golden_kivi_stage2(g):
    f = load("kivi_qk_ref")
    s, i = osel.kivi_qk_dense_sparse(**stage2_inputs(f, g))
    check_stage2_against_golden(s, i, f, g)


def check_quest_against_golden(ours, f):
    """fp32 scores with exact products (CUDA semantics) against QuestPytorch's."""
    q = bf16_to_f32(f["raw_q"])
    mn, mx = bf16_to_f32(f["chunk_min"]), bf16_to_f32(f["chunk_max"])
    n = int(f["n_chunks"])
    v = f["valid"][:, :, :n]
    ref = f["scores"]
    # invalid chunks: torch fills finfo(bf16).min, the CUDA kernel -inf
    assert np.all(ref[~v] == np.float32(-3.3895313892515355e38)) and np.all(np.isneginf(ours[~v]))
    qq = q[:, :, None, :]
    m = np.maximum(qq * mn[:, :, :n], qq * mx[:, :, :n])
    bound = np.abs(m).sum(-1) * 2.0 ** -9 + bf16_ulp(ref) / 2 + 1e-6
    err = np.abs(ours[v] - ref[v])
    assert np.all(err <= bound[v]), float((err - bound[v]).max())
    # the torch value is itself the bf16 rounding of its own sum
    assert np.array_equal(bf16r(ref[v]), ref[v])


def test_golden_quest_torch():
    f = load("quest_torch")
    ours = osel.quest_chunk_score(bf16_to_f32(f["raw_q"]), bf16_to_f32(f["chunk_min"]),
                                  bf16_to_f32(f["chunk_max"]), int(f["n_chunks"]), f["valid"])
    check_quest_against_golden(ours, f)


def test_golden_lse_merge_torch():
    f = load("lse_merge_torch")
    la, lb = f["lse_a"][..., 0], f["lse_b"][..., 0]
    ours = okivi.lse_merge(f["a"][:, 0], la, f["b"][:, 0], lb)
    ref = f["merged_f32"][:, 0]
    assert np.abs(ours - ref).max() <= 4e-6 * (1 + np.abs(ours).max())
    ours_b = okivi.lse_merge(bf16_to_f32(f["a_bf16"])[:, 0], la, bf16_to_f32(f["b_bf16"])[:, 0], lb)
    ref_b = bf16_to_f32(f["merged_bf16"])[:, 0]
    assert np.all(np.abs(bf16r(ours_b) - ref_b) <= bf16_ulp(ref_b))
    # the far-apart pair takes (almost) all its weight from b
    assert np.allclose(ref[0, 0], f["b"][0, 0, 0], atol=1e-6)
