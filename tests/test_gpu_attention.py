"""GPU parity of the bf16 K/V decode attention (flash_attn_with_kvcache_compat
counterpart) and the LSE merge (lse_merge_torch counterpart) against the
float64 oracle; outputs within 2e-3, LSEs within 1e-4 relative."""
import numpy as np
import pytest
import torch

from oracle import kivi as okivi
from tests.helpers import from_torch, gaussian_bf16, to_bf16

pytestmark = pytest.mark.gpu

ATOL = 2e-3


@pytest.mark.parametrize("bs,hq,kv,n,splits", [
    (2, 32, 8, 420, 0),      # sink + local + selected tokens of the reference's sparse path
    (1, 32, 8, 930, 0),
    (3, 8, 2, 1, 0),         # a single key
    (2, 8, 2, 33, 1),
    (1, 16, 1, 2000, 3),
    (2, 4, 4, 100, 0),       # MHA
])
def test_bf16_attention_matches_oracle(rng, bs, hq, kv, n, splits):
    from zoomkv_revision_amd.attention import flash_attn_with_kvcache_compat
    q = gaussian_bf16(rng, (bs, hq, 128))
    k = gaussian_bf16(rng, (bs, kv, n, 128), outlier_channels=2)
    v = gaussian_bf16(rng, (bs, kv, n, 128))
    # the reference hands over concat(...).transpose(1, 2): [bs, n, kv, 128] views
    kt, vt = to_bf16(k).transpose(1, 2), to_bf16(v).transpose(1, 2)
    out, lse = flash_attn_with_kvcache_compat(to_bf16(q).unsqueeze(1), kt, vt, causal=False,
                                              return_softmax_lse=True, n_splits=splits)
    ref, rlse = okivi.attention(q, k, v, 1 / np.sqrt(128), return_lse=True)
    got = from_torch(out)[:, 0]
    assert out.shape == (bs, 1, hq, 128) and lse.shape == (bs, hq, 1)
    assert np.abs(got - ref).max() <= ATOL + np.abs(ref).max() * 2 ** -8
    assert np.allclose(from_torch(lse)[..., 0], rlse, rtol=1e-4, atol=1e-4)


def test_bf16_attention_contiguous_layout_and_scale(rng):
    from zoomkv_revision_amd.attention import flash_attn_with_kvcache_compat
    q = gaussian_bf16(rng, (2, 8, 128))
    k = gaussian_bf16(rng, (2, 77, 2, 128))            # contiguous [bs, n, kv, 128]
    v = gaussian_bf16(rng, (2, 77, 2, 128))
    out = flash_attn_with_kvcache_compat(to_bf16(q).unsqueeze(1), to_bf16(k), to_bf16(v),
                                         softmax_scale=0.05)
    ref = okivi.attention(q, np.swapaxes(k, 1, 2), np.swapaxes(v, 1, 2), 0.05)
    assert np.abs(from_torch(out)[:, 0] - ref).max() <= ATOL + np.abs(ref).max() * 2 ** -8
    with pytest.raises(NotImplementedError):
        flash_attn_with_kvcache_compat(to_bf16(q).unsqueeze(1), to_bf16(k), to_bf16(v), cache_seqlens=3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("lse_shape", ["bh1", "b1h", "bh"])
def test_lse_merge_matches_oracle(rng, dtype, lse_shape):
    from zoomkv_revision_amd.attention import lse_merge_torch
    bs, h, d = 3, 32, 128
    a = rng.standard_normal((bs, 1, h, d)).astype(np.float32)
    b = rng.standard_normal((bs, 1, h, d)).astype(np.float32)
    la = (rng.standard_normal((bs, h)) * 4).astype(np.float32)
    lb = (rng.standard_normal((bs, h)) * 4).astype(np.float32)
    ta, tb = torch.from_numpy(a).cuda().to(dtype), torch.from_numpy(b).cuda().to(dtype)
    shp = {"bh1": lambda x: x[..., None], "b1h": lambda x: x[:, None], "bh": lambda x: x}[lse_shape]
    got = lse_merge_torch(ta, torch.from_numpy(shp(la)).cuda(), tb, torch.from_numpy(shp(lb)).cuda())
    assert got.dtype == dtype and got.shape == (bs, 1, h, d)
    ref = okivi.lse_merge(ta.float().cpu().numpy()[:, 0], la, tb.float().cpu().numpy()[:, 0], lb)
    tol = {torch.bfloat16: 2 ** -8, torch.float16: 2 ** -11, torch.float32: 1e-6}[dtype]
    assert np.abs(got.float().cpu().numpy()[:, 0] - ref).max() <= tol * (1 + np.abs(ref).max())


def test_split_attention_merged_by_lse_equals_full(rng):
    """Two segments attended separately and merged by LSE equal one attention
    over both (the context-sharded decode: partial (o, lse) per shard)."""
    from zoomkv_revision_amd.attention import flash_attn_with_kvcache_compat, lse_merge
    q = to_bf16(gaussian_bf16(rng, (2, 32, 128))).unsqueeze(1)
    k = to_bf16(gaussian_bf16(rng, (2, 300, 8, 128)))
    v = to_bf16(gaussian_bf16(rng, (2, 300, 8, 128)))
    oa, la = flash_attn_with_kvcache_compat(q, k[:, :130], v[:, :130], return_softmax_lse=True)
    ob, lb = flash_attn_with_kvcache_compat(q, k[:, 130:], v[:, 130:], return_softmax_lse=True)
    fa32 = lambda x: x.float().cpu().numpy()
    merged = okivi.lse_merge(fa32(oa)[:, 0], fa32(la)[..., 0], fa32(ob)[:, 0], fa32(lb)[..., 0])
    full = fa32(flash_attn_with_kvcache_compat(q, k, v))[:, 0]
    assert np.abs(merged - full).max() <= ATOL
    assert np.abs(fa32(lse_merge(oa, la, ob, lb))[:, 0] - full).max() <= ATOL


@pytest.mark.parametrize("n_idx,tail_start,tail_len", [(100, 300, 40), (0, 10, 77), (64, 0, 0), (5, 499, 1)])
def test_gather_attention_matches_gathered_oracle(rng, n_idx, tail_start, tail_len):
    """Index list (with invalid ids masked) + contiguous tail == gather, cat,
    attend (the reference's compute() tail)."""
    from zoomkv_revision_amd.attention import gather_attention
    bs, hq, kv, rows = 2, 32, 8, 500
    q = gaussian_bf16(rng, (bs, hq, 128))
    k = gaussian_bf16(rng, (bs, kv, rows, 128))
    v = gaussian_bf16(rng, (bs, kv, rows, 128))
    idx = rng.integers(0, rows, size=(bs, kv, n_idx))
    if n_idx > 3:
        idx[0, 1, 2] = -1           # masked
        idx[1, 3, 0] = rows + 7     # masked
    out, lse = gather_attention(to_bf16(q).unsqueeze(1), to_bf16(k), to_bf16(v),
                                torch.from_numpy(idx).cuda() if n_idx else None, tail_start, tail_len,
                                return_softmax_lse=True)
    ref = np.zeros((bs, hq, 128))
    rlse = np.zeros((bs, hq))
    g = hq // kv
    for b in range(bs):
        for h in range(kv):
            sel = [r for r in idx[b, h] if 0 <= r < rows] + list(range(tail_start, tail_start + tail_len))
            o, l = okivi.attention(q[b:b + 1, h * g:(h + 1) * g], k[b, h, sel][None, None], v[b, h, sel][None, None],
                                   1 / np.sqrt(128), return_lse=True)
            ref[b, h * g:(h + 1) * g], rlse[b, h * g:(h + 1) * g] = o[0], l[0]
    assert np.abs(from_torch(out)[:, 0] - ref).max() <= ATOL + np.abs(ref).max() * 2 ** -8
    assert np.allclose(from_torch(lse)[..., 0], rlse, rtol=1e-4, atol=1e-4)
