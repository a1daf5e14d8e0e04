"""The allocation-free decode attention (zkv_kivi4_decode_attention_noalloc,
split partials in the library's static per-GPU scratch) through the C ABI:
two calls in a row, the second with a smaller input, each equal to
zkv_kivi4_decode_attention's output with a caller workspace; a split plan
beyond the static scratch is rejected without a launch."""
import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import gaussian_bf16, to_bf16

pytestmark = pytest.mark.gpu


def _case(rng, bs, hq, kv, ng, res):
    from zoomkv_revision_amd import kivi
    cache = kivi.Kivi4Cache.allocate(bs, kv, ng, max(res, 1))
    k = gaussian_bf16(rng, (bs, kv, ng * 32, 128), outlier_channels=1)
    v = gaussian_bf16(rng, (bs, kv, ng * 32, 128))
    kivi.kivi4_pack(to_bf16(k), to_bf16(v), cache, 0)
    if res:
        cache.k_res[:, :, :res].copy_(to_bf16(gaussian_bf16(rng, (bs, kv, res, 128))))
        cache.v_res[:, :, :res].copy_(to_bf16(gaussian_bf16(rng, (bs, kv, res, 128))))
    q = to_bf16(gaussian_bf16(rng, (bs, hq, 128)))
    return cache, q


def _args(q, cache, ng, res, hq, kv, out):
    return (q.data_ptr(), q.stride(0), q.stride(1), cache.groups.data_ptr(), cache.g_cap,
            cache.k_res.data_ptr(), cache.v_res.data_ptr(), cache.r_cap, q.shape[0], hq, kv, ng, res,
            1.0 / np.sqrt(128), out.data_ptr(), 1, None)


def test_noalloc_attention_equals_workspace_attention_twice(rng):
    from zoomkv_revision_amd._lib import lib
    L = lib()
    stream = torch.cuda.current_stream().cuda_stream
    for bs, hq, kv, ng, res, splits in ((4, 32, 8, 60, 50, 0), (2, 16, 4, 9, 17, 3)):
        cache, q = _case(rng, bs, hq, kv, ng, res)
        ref = torch.empty(bs, hq, 128, dtype=torch.float32, device="cuda")
        got = torch.full((bs, hq, 128), float("nan"), dtype=torch.float32, device="cuda")
        n = L.zkv_kivi4_attention_workspace_size(bs, hq, kv, ng, res, splits)
        ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        rc = L.zkv_kivi4_decode_attention(*_args(q, cache, ng, res, hq, kv, ref), splits, ws.data_ptr(), n, stream)
        assert rc == 0, L.zkv_last_error()
        rc = L.zkv_kivi4_decode_attention_noalloc(*_args(q, cache, ng, res, hq, kv, got), splits, stream)
        assert rc == 0, L.zkv_last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref), (bs, hq, kv, ng, res, (got - ref).abs().max().item())


def test_noalloc_attention_rejects_plans_beyond_the_scratch(rng):
    from zoomkv_revision_amd._lib import lib
    L = lib()
    bs, hq, kv, ng = 16, 32, 8, 64
    cache, q = _case(rng, bs, hq, kv, ng, 0)
    out = torch.zeros(bs, hq, 128, dtype=torch.float32, device="cuda")
    # 40 splits: 16 x 32 x 40 x 520 bytes of partials > 8 MiB
    rc = L.zkv_kivi4_decode_attention_noalloc(*_args(q, cache, ng, 0, hq, kv, out), 40,
                                              torch.cuda.current_stream().cuda_stream)
    assert rc == 3 and b"static scratch" in L.zkv_last_error()
    torch.cuda.synchronize()
    assert not out.any()                                       # nothing was launched
