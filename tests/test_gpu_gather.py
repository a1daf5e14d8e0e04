"""GPU: host-to-device row gather from pinned host memory (the reference's
trans_h2d.py:65-166; its own check, trans_h2d.py:168-200, compares against
src.cuda()[b][h][indices] -- done here row by row, bit-exact)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _pinned(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.bfloat16).pin_memory()


def test_h2d_gather_kv_matches_indexing():
    from zoomkv_revision_amd.gather import h2d_gather_kv
    bs, heads, kv_len, topk, max_topk = 2, 8, 4096, 100, 160
    sk, sv = _pinned((bs, heads, kv_len, 128), 1), _pinned((bs, heads, kv_len, 128), 2)
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, kv_len, (bs, heads, topk), generator=g)
    idx[0, 0, 5] = -1                      # out of range: row left untouched
    idx[1, 3, 7] = kv_len
    dk = torch.full((bs, heads, max_topk, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    dv = torch.full_like(dk, -3.0)
    h2d_gather_kv(sk, sv, idx.cuda(), dk, dv)
    torch.cuda.synchronize()
    ref_k = sk.clone()
    ok = (idx >= 0) & (idx < kv_len)
    gk, gv = dk.cpu(), dv.cpu()
    for b in range(bs):
        for h in range(heads):
            for j in range(topk):
                if ok[b, h, j]:
                    assert torch.equal(gk[b, h, j], ref_k[b, h, idx[b, h, j]])
                    assert torch.equal(gv[b, h, j], sv[b, h, idx[b, h, j]])
                else:
                    assert torch.all(gk[b, h, j] == 7.0) and torch.all(gv[b, h, j] == -3.0)
    assert torch.all(gk[:, :, topk:] == 7.0)


def test_h2d_gather_kv_packed_segments():
    from zoomkv_revision_amd.gather import h2d_gather_kv_packed
    bs, kvh, src_len, sl_end = 2, 3, 2048, 5
    sk, sv = _pinned((bs, kvh, src_len, 128), 4), _pinned((bs, kvh, src_len, 128), 5)
    g = torch.Generator().manual_seed(6)
    ks = [int(x) for x in torch.randint(0, 40, (bs * kvh,), generator=g)]
    cu_topk = np.concatenate([[0], np.cumsum(ks)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum([k + sl_end for k in ks])]).astype(np.int32)
    idx = torch.randint(0, src_len, (int(cu_topk[-1]),), generator=g)
    total_k = int(cu_k[-1])
    dk = torch.zeros(total_k, 128, dtype=torch.bfloat16, device="cuda")
    dv = torch.zeros_like(dk)
    h2d_gather_kv_packed(sk, sv, dk, dv, idx.cuda(), torch.from_numpy(cu_topk).cuda(),
                         torch.from_numpy(cu_k).cuda(), sl_end, max(ks))
    torch.cuda.synchronize()
    gk, gv = dk.cpu(), dv.cpu()
    for vh in range(bs * kvh):
        b, h = divmod(vh, kvh)
        assert torch.all(gk[cu_k[vh]:cu_k[vh] + sl_end] == 0)       # the caller's rows untouched
        for s in range(ks[vh]):
            i = int(idx[cu_topk[vh] + s])
            assert torch.equal(gk[cu_k[vh] + sl_end + s], sk[b, h, i])
            assert torch.equal(gv[cu_k[vh] + sl_end + s], sv[b, h, i])


def test_h2d_gather_rejects_unpinned_source():
    from zoomkv_revision_amd.gather import h2d_gather_kv
    src = torch.zeros(1, 1, 16, 128, dtype=torch.bfloat16)
    dst = torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16, device="cuda")
    idx = torch.zeros(1, 1, 4, dtype=torch.int64, device="cuda")
    with pytest.raises(AssertionError):
        h2d_gather_kv(src, src, idx, dst, dst)


def test_h2d_gather_c_abi_reports_unmapped_host_memory():
    """Through the C ABI: a host buffer with no device alias is an error, not a fault."""
    from zoomkv_revision_amd._lib import lib
    src = np.zeros((1, 1, 16, 128), dtype=np.uint16)               # ordinary pageable memory
    dst = torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16, device="cuda")
    idx = torch.zeros(1, 1, 4, dtype=torch.int64, device="cuda")
    rc = lib().zkv_h2d_gather_kv(src.ctypes.data, src.ctypes.data, 1, 1, 16, idx.data_ptr(), 4,
                                 dst.data_ptr(), dst.data_ptr(), 4, torch.cuda.current_stream().cuda_stream)
    assert rc == 1 and b"not pinned" in lib().zkv_last_error()


def test_copy_rows_between_device_and_pinned_host_rows():
    """The offload flush's pitched copy: device staging [bs, kv, n, 128] into
    rows [w0, w0 + n) of a pinned host [bs, kv, cap, 128], and back."""
    from zoomkv_revision_amd.gather import copy_rows
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    stage = torch.randn(3, 4, 48, 128, generator=g, device="cuda").to(torch.bfloat16)
    host = torch.zeros(3, 4, 100, 128, dtype=torch.bfloat16, pin_memory=True)
    copy_rows(host[:, :, 17:17 + 40], stage[:, :, :40])
    torch.cuda.synchronize()
    assert torch.equal(host[:, :, 17:57], stage[:, :, :40].cpu())
    assert not host[:, :, :17].any() and not host[:, :, 57:].any()
    back = torch.zeros(3, 4, 40, 128, dtype=torch.bfloat16, device="cuda")
    copy_rows(back, host[:, :, 17:57])
    torch.cuda.synchronize()
    assert torch.equal(back, stage[:, :, :40])


def test_pinned_empty_is_pinned_gatherable_and_released():
    """Exact-size pinned host tensors: torch sees them as pinned, the h2d
    gather reads them, and dropping the last view releases the memory (72
    rounds of 1 GiB pass only if each is freed: the host pins about 65 GiB)."""
    import gc
    from zoomkv_revision_amd.gather import h2d_gather_kv, pinned_empty
    k = pinned_empty((2, 3, 50, 128), torch.bfloat16)
    v = pinned_empty((2, 3, 50, 128), torch.bfloat16)
    assert k.is_pinned() and v.is_pinned() and k.shape == (2, 3, 50, 128)
    k.copy_(torch.arange(2 * 3 * 50 * 128, dtype=torch.float32).view(2, 3, 50, 128))
    v.copy_(-k.float())
    idx = torch.tensor([[[4, 49, 0]] * 3] * 2, dtype=torch.int64, device="cuda")
    dk = torch.zeros(2, 3, 3, 128, dtype=torch.bfloat16, device="cuda")
    dv = torch.zeros_like(dk)
    h2d_gather_kv(k[:, :, :50], v, idx, dk, dv)
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), k[:, :, [4, 49, 0]]) and torch.equal(dv.cpu(), v[:, :, [4, 49, 0]])
    view = k[1, 2]
    del k
    gc.collect()
    assert view.sum().item() != 0                   # a view keeps the block alive
    del view, v
    for _ in range(72):
        t = pinned_empty((1 << 30,), torch.uint8)
        t[::1 << 20] = 1
        del t
        gc.collect()
