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


@pytest.mark.parametrize("bs,hq,kv,n,splits", [(2, 32, 8, 420, 0), (1, 32, 8, 930, 0), (1, 16, 1, 2000, 3),
                                               (3, 8, 2, 1, 0)])
def test_bf16_attention_fp32_output_strict(rng, bs, hq, kv, n, splits):
    """The unrounded (fp32) output of flash_attn_with_kvcache_compat within the
    north star's 2e-3 of the float64 oracle, with no bf16 output slack."""
    from zoomkv_revision_amd.attention import flash_attn_with_kvcache_compat
    q = gaussian_bf16(rng, (bs, hq, 128))
    k = gaussian_bf16(rng, (bs, kv, n, 128), outlier_channels=2)
    v = gaussian_bf16(rng, (bs, kv, n, 128))
    out = torch.empty(bs, 1, hq, 128, dtype=torch.float32, device="cuda")
    flash_attn_with_kvcache_compat(to_bf16(q).unsqueeze(1), to_bf16(k).transpose(1, 2),
                                   to_bf16(v).transpose(1, 2), out=out, n_splits=splits)
    ref = okivi.attention(q, k, v, 1 / np.sqrt(128))
    err = np.abs(from_torch(out)[:, 0] - ref).max()
    assert err <= ATOL, f"max abs err {err}"


@pytest.mark.parametrize("n_idx,tail_start,tail_len", [(100, 300, 40), (612, 400, 100)])
def test_gather_attention_fp32_output_strict(rng, n_idx, tail_start, tail_len):
    from zoomkv_revision_amd.attention import gather_attention
    bs, hq, kv, rows = 2, 32, 8, 1000
    q = gaussian_bf16(rng, (bs, hq, 128))
    k = gaussian_bf16(rng, (bs, kv, rows, 128), outlier_channels=2)
    v = gaussian_bf16(rng, (bs, kv, rows, 128))
    idx = rng.integers(0, rows, size=(bs, kv, n_idx))
    out = torch.empty(bs, 1, hq, 128, dtype=torch.float32, device="cuda")
    gather_attention(to_bf16(q).unsqueeze(1), to_bf16(k), to_bf16(v), torch.from_numpy(idx).cuda(),
                     tail_start, tail_len, out=out)
    g = hq // kv
    ref = np.zeros((bs, hq, 128))
    for b in range(bs):
        for h in range(kv):
            sel = list(idx[b, h]) + list(range(tail_start, tail_start + tail_len))
            ref[b, h * g:(h + 1) * g] = okivi.attention(q[b:b + 1, h * g:(h + 1) * g], k[b, h, sel][None, None],
                                                        v[b, h, sel][None, None], 1 / np.sqrt(128))[0]
    err = np.abs(from_torch(out)[:, 0] - ref).max()
    assert err <= ATOL, f"max abs err {err}"


def test_bf16_attention_values_beyond_fp16(rng):
    """bf16 K / V enter the bf16 matrix cores unconverted: values far outside
    fp16's range (|K| up to 3e5, |V| up to 7e4) give finite outputs that match
    the float64 oracle to 2e-3 relative to the value scale."""
    from zoomkv_revision_amd.attention import flash_attn_with_kvcache_compat
    from oracle.numerics import bf16r
    bs, hq, kv, n = 2, 16, 4, 300
    q = gaussian_bf16(rng, (bs, hq, 128))
    k = gaussian_bf16(rng, (bs, kv, n, 128))
    v = gaussian_bf16(rng, (bs, kv, n, 128))
    k[0, 1, 17, 5] = bf16r(np.float32(3.0e5))      # one token's key far outside fp16
    k[1, 2, 200, 9] = bf16r(np.float32(-9.0e4))
    v[0, 1, 17, :] = bf16r(np.linspace(-7.0e4, 7.0e4, 128, dtype=np.float32))
    v[1, 3, 33, 40] = bf16r(np.float32(1.0e5))
    out = torch.empty(bs, 1, hq, 128, dtype=torch.float32, device="cuda")
    flash_attn_with_kvcache_compat(to_bf16(q).unsqueeze(1), to_bf16(k).transpose(1, 2),
                                   to_bf16(v).transpose(1, 2), out=out)
    got = from_torch(out)[:, 0]
    ref = okivi.attention(q, k, v, 1 / np.sqrt(128))
    assert np.isfinite(got).all()
    scale = np.maximum(1.0, np.abs(ref).max(axis=-1, keepdims=True))        # per (batch, query head)
    assert np.all(np.abs(got - ref) <= ATOL * scale)
