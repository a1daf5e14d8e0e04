"""The gfx950 kernels against the golden vectors written by the reference's
own pure-PyTorch functions (tests/golden/make_golden.py), through the C ABI:
chunk statistics + Format R pack bit-exact with quant_pack.py / S:2133-2135 /
S:2017, the stage-2 scorer and Quest within the rounding gap stated in
tests/test_golden.py, and lse_merge within fp32 / bf16 rounding."""
import numpy as np
import pytest
import torch

from oracle.numerics import bf16_to_f32, bf16r
from tests.test_golden import (bf16_ulp, check_quest_against_golden, check_stage2_against_golden,
                               load)

pytestmark = pytest.mark.gpu

DEV = "cuda"


def bf16_dev(u16: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(u16.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16).to(DEV)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("g", [8, 16])
def test_gpu_golden_chunk_encode(g):
    from zoomkv_revision_amd import kivi
    f = load("kivi_quant_pack")
    keys = bf16_dev(f["K"])
    bs, kv, n, _ = keys.shape
    nc = n // g
    n_max = nc + 2
    mn = torch.zeros(bs, kv, n_max, 128, dtype=torch.bfloat16, device=DEV)
    mx, mean = torch.zeros_like(mn), torch.zeros_like(mn)
    valid = torch.zeros(bs, kv, n_max, dtype=torch.bool, device=DEV)
    packed = torch.zeros(bs, kv, n_max, 16, g, dtype=torch.int32, device=DEV)
    assert kivi.chunk_encode(keys, g, 0, mn, mx, mean, valid, packed) == nc
    torch.cuda.synchronize()
    assert np.array_equal(bits_of(mn[:, :, :nc]), f[f"g{g}_min"])
    assert np.array_equal(bits_of(mx[:, :, :nc]), f[f"g{g}_max"])
    assert np.array_equal(bits_of(mean[:, :, :nc]), f[f"g{g}_mean"])
    assert np.array_equal(packed[:, :, :nc].cpu().numpy(), f[f"g{g}_packed_cm"])
    assert valid[:, :, :nc].all() and not valid[:, :, nc:].any()


@pytest.mark.parametrize("g", [16, 8])
def test_gpu_golden_kivi_stage2(g):
    from zoomkv_revision_amd import kivi
    f = load("kivi_qk_ref")
    ids = torch.from_numpy(f[f"g{g}_chunk_ids"]).to(DEV)
    mask = torch.from_numpy(f[f"g{g}_dense_mask"]).to(DEV)
    packed = torch.from_numpy(f[f"g{g}_packed_cm"]).to(DEV)
    dense, sparse = (int(x) for x in f[f"g{g}_topk"])
    bs, kv, nk = ids.shape
    s = torch.empty(bs, kv, nk * g, dtype=torch.float32, device=DEV)
    i = torch.empty(bs, kv, nk * g, dtype=torch.int64, device=DEV)
    kivi.partial_chunk_kivi_qk_dense_sparse_cuda(ids, mask, packed, bf16_dev(f[f"g{g}_min"]),
                                                 bf16_dev(f[f"g{g}_max"]), bf16_dev(f[f"g{g}_raw_q"]),
                                                 dense, sparse, g, s, i)
    torch.cuda.synchronize()
    check_stage2_against_golden(s.cpu().numpy(), i.cpu().numpy(), f, g)


def test_gpu_golden_quest():
    from zoomkv_revision_amd import quest
    f = load("quest_torch")
    q = bf16_dev(f["raw_q"])
    bs, kv, _ = q.shape
    n = int(f["n_chunks"])
    scores = torch.empty(bs, kv, n, dtype=torch.float32, device=DEV)
    quest.quest_chunk_score(q, bf16_dev(f["chunk_min"]), bf16_dev(f["chunk_max"]), scores, n,
                            torch.from_numpy(f["valid"]).to(DEV))
    torch.cuda.synchronize()
    check_quest_against_golden(scores.cpu().numpy(), f)


def test_gpu_golden_lse_merge():
    from zoomkv_revision_amd.attention import lse_merge_torch
    f = load("lse_merge_torch")
    la = torch.from_numpy(f["lse_a"]).to(DEV)
    lb = torch.from_numpy(f["lse_b"]).to(DEV)
    out = lse_merge_torch(torch.from_numpy(f["a"]).to(DEV), la, torch.from_numpy(f["b"]).to(DEV), lb)
    ref = f["merged_f32"]
    assert out.dtype == torch.float32
    assert np.abs(out.cpu().numpy() - ref).max() <= 4e-6 * (1 + np.abs(ref).max())
    out_b = lse_merge_torch(bf16_dev(f["a_bf16"]), la, bf16_dev(f["b_bf16"]), lb)
    ref_b = bf16_to_f32(f["merged_bf16"])
    got_b = out_b.float().cpu().numpy()
    assert out_b.dtype == torch.bfloat16
    assert np.all(np.abs(bf16r(got_b) - ref_b) <= bf16_ulp(ref_b))
