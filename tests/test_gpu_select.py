"""GPU parity of the page-scoring / selection kernels against the CPU oracle
(bit-exact scores, indices and masks)."""
import numpy as np
import pytest
import torch

from oracle import select as osel
from oracle.kivi import encode_chunks_ref
from oracle.numerics import bf16r, f16_bits, f16_to_f32
from tests.helpers import from_torch, gaussian_bf16, to_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fp16_meta", [False, True])
def test_quest_chunk_score_bit_exact(rng, fp16_meta):
    from zoomkv_revision_amd.quest import load_kernel_module
    bs, kv, n_max, n = 2, 3, 40, 37
    k = gaussian_bf16(rng, (bs, kv, n_max * 16, 128), outlier_channels=4)
    mn, mx, _, _ = encode_chunks_ref(k, 16)
    if fp16_meta:
        mn, mx = f16_to_f32(f16_bits(mn)), f16_to_f32(f16_bits(mx))
    q = gaussian_bf16(rng, (bs, kv, 128))
    valid = rng.random((bs, kv, n_max)) > 0.1
    ref = osel.quest_chunk_score(q, mn, mx, n, valid)
    dt = torch.float16 if fp16_meta else torch.bfloat16
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dt)
    scores = torch.empty(bs, kv, n, dtype=torch.float32, device="cuda")
    load_kernel_module().quest_chunk_score(to_bf16(q), t(mn), t(mx), scores, n,
                                           torch.from_numpy(valid).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(scores).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("fp16_meta,bs,hq,kv,n_max,n,four_dim", [
    (False, 2, 32, 8, 40, 37, True),     # the cache's [bs, 1, hq, 128] queries
    (True, 3, 8, 2, 9, 9, False),
    (False, 2, 6, 6, 5, 1, False),       # one chunk per (b, h): every chunk of a trip changes (b, h)
    (False, 1, 16, 2, 8, 3, True),       # 3 chunks: trips straddle (b, h)
    (True, 4, 32, 4, 600, 523, False),
    (False, 1, 32, 2, 50, 50, False),    # 16 query heads per KV head: rows past the first 8 summed one by one
])
def test_quest_chunk_score_gqa_bit_exact(rng, fp16_meta, bs, hq, kv, n_max, n, four_dim):
    """The fused launch equals the GQA-mean kernel followed by the Quest scan:
    raw_q bit-exact with the torch-mean restatement, scores bit-exact."""
    from zoomkv_revision_amd.quest import quest_chunk_score_gqa
    k = gaussian_bf16(rng, (bs, kv, n_max * 16, 128), outlier_channels=4)
    mn, mx, _, _ = encode_chunks_ref(k, 16)
    if fp16_meta:
        mn, mx = f16_to_f32(f16_bits(mn)), f16_to_f32(f16_bits(mx))
    q = gaussian_bf16(rng, (bs, hq, 128))
    valid = rng.random((bs, kv, n_max)) > 0.1
    raw_ref = osel.gqa_mean_query(q, kv)
    ref = osel.quest_chunk_score(raw_ref, mn, mx, n, valid)
    dt = torch.float16 if fp16_meta else torch.bfloat16
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dt)
    qt = to_bf16(q)
    if four_dim:
        qt = qt.unsqueeze(1)
    scores = torch.empty(bs, kv, n, dtype=torch.float32, device="cuda")
    raw_q = torch.full((bs, kv, 128), 7.0, dtype=torch.bfloat16, device="cuda")
    quest_chunk_score_gqa(qt, kv, t(mn), t(mx), scores, n, torch.from_numpy(valid).cuda(), raw_q)
    torch.cuda.synchronize()
    assert np.array_equal(from_torch(raw_q), raw_ref)
    assert np.array_equal(from_torch(scores).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("L,k", [(2048, 128), (13120, 100), (131072, 256), (64, 64), (3000, 1),
                                 (4096, 1638), (1638, 491), (26208, 100), (32768, 7), (32769, 300),
                                 # register-bucket edges (1024 * R) and k = L - 1
                                 (4096, 4095), (4097, 5), (8192, 8191), (8193, 64), (16384, 1),
                                 (16385, 2048), (1025, 1024)])
def test_topk_exact(rng, L, k):
    from zoomkv_revision_amd.topk import float_topk_3d
    x = rng.standard_normal((2, 3, L)).astype(np.float32)
    x[0, 0, ::7] = 1.5                          # heavy ties
    x[1, 2, : L // 2] = x[1, 2, 0]              # a tie block bigger than k
    got = from_torch(float_topk_3d(torch.from_numpy(x).cuda(), k))
    assert np.array_equal(got, osel.topk_indices(x, k))


def test_topk_rejects_k_above_length():
    # float_topk_ops.py:103 asserts k <= n_chunks before launching
    from zoomkv_revision_amd.topk import float_topk_3d
    with pytest.raises(AssertionError):
        float_topk_3d(torch.zeros(1, 1, 50, device="cuda"), 64)


def test_topk_strided_and_bf16_input(rng):
    from zoomkv_revision_amd.topk import float_topk, float_topk_3d
    x = rng.standard_normal((4, 5, 300)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    assert np.array_equal(from_torch(float_topk_3d(xt[:, 1:4], 17)), osel.topk_indices(x[:, 1:4], 17))
    # rows that are not 16-byte aligned (scalar loads)
    y = rng.standard_normal((3, 9001)).astype(np.float32)
    yt = torch.from_numpy(y).cuda()
    assert np.array_equal(from_torch(float_topk(yt[:, 1:], 40)), osel.topk_indices(y[:, 1:], 40))
    xb = bf16r(x[0])
    assert np.array_equal(from_torch(float_topk(to_bf16(xb), 9)), osel.topk_indices(xb, 9))


def test_topk_gather_concat(rng):
    from zoomkv_revision_amd.topk import float_topk_gather_concat_3d
    bs, kv, L, k, sk = 2, 4, 1600, 100, 5
    sc = rng.standard_normal((bs, kv, L)).astype(np.float32)
    lut = rng.integers(0, 10 ** 6, size=(bs, kv, L))
    skipped = rng.integers(0, 99, size=(bs, kv, sk))
    out = torch.full((bs, kv, 612), -7, dtype=torch.int64, device="cuda")
    float_topk_gather_concat_3d(torch.from_numpy(sc).cuda(), torch.from_numpy(lut).cuda(),
                                torch.from_numpy(skipped).cuda(), out, k)
    got = from_torch(out)
    ref = osel.topk_gather_concat(sc, lut, skipped, k, k + sk)
    assert np.array_equal(got[..., :k + sk], ref)
    assert np.all(got[..., k + sk:] == -7)
    # L <= k (reachable through the C ABI; the Python wrappers assert k <= L
    # like the reference's): lut prefix, skipped tail after k, 0 sentinel
    from zoomkv_revision_amd._lib import check, lib, ptr, stream_of
    sc2 = torch.ones(1, 3, device="cuda")
    lut2 = torch.tensor([[5, 6, 7]], device="cuda")
    sk2 = torch.tensor([[41, 42]], device="cuda")
    out2 = torch.full((1, 10), -7, dtype=torch.int64, device="cuda")
    check(lib().zkv_topk(ptr(sc2), 3, 1, 3, 6, ptr(out2), 10, ptr(lut2), 3, ptr(sk2), 2, 2, 0,
                         stream_of(sc2)))
    assert from_torch(out2)[0].tolist() == [5, 6, 7, 0, 0, 0, 41, 42, -7, -7]
    out3 = torch.full((1, 6), -7, dtype=torch.int64, device="cuda")
    check(lib().zkv_topk(ptr(sc2), 3, 1, 3, 5, ptr(out3), 6, None, 0, None, 0, 0, -1, stream_of(sc2)))
    assert from_torch(out3)[0].tolist() == [0, 1, 2, -1, -1, -7]


def test_density_and_mask_bit_exact(rng):
    from zoomkv_revision_amd.rerank import dense_mask_from_topk_cuda, partial_chunk_density_scores_cuda
    bs, kv, n, nk = 2, 3, 50, 21
    cent = gaussian_bf16(rng, (bs, kv, n, 128))
    q = gaussian_bf16(rng, (bs, kv, 128))
    ids = rng.integers(-2, n + 2, size=(bs, kv, nk))
    out = torch.empty(bs, kv, nk, dtype=torch.float32, device="cuda")
    partial_chunk_density_scores_cuda(torch.from_numpy(ids).cuda(), to_bf16(cent), to_bf16(q), out)
    ref = osel.chunk_density_scores(ids, cent, q)
    assert np.array_equal(from_torch(out).view(np.uint32), ref.view(np.uint32))
    pos = rng.integers(-1, nk + 1, size=(bs, kv, 6))
    mask = torch.ones(bs, kv, nk, dtype=torch.bool, device="cuda")
    dense_mask_from_topk_cuda(torch.from_numpy(pos).cuda(), mask)
    assert np.array_equal(from_torch(mask), osel.dense_mask_from_topk(pos, nk))


def test_gqa_mean_bit_exact(rng):
    from zoomkv_revision_amd.rerank import gqa_mean_query
    q = gaussian_bf16(rng, (3, 32, 128))
    got = gqa_mean_query(to_bf16(q).unsqueeze(1), 8)
    assert np.array_equal(from_torch(got), osel.gqa_mean_query(q, 8))


@pytest.mark.parametrize("g", [8, 16])
def test_kivi_qk_dense_sparse_bit_exact(rng, g):
    from zoomkv_revision_amd.kivi import partial_chunk_kivi_qk_dense_sparse_cuda
    bs, kv, n_chunks, nk = 2, 3, 60, 37
    keys = gaussian_bf16(rng, (bs, kv, n_chunks * g, 128), outlier_channels=4)
    mn, mx, _, packed = encode_chunks_ref(keys, g)
    q = gaussian_bf16(rng, (bs, kv, 128))
    ids = rng.integers(0, n_chunks, size=(bs, kv, nk))
    ids[0, 1, 3] = n_chunks + 5                       # out of range -> -1e30 slots
    dm = rng.random((bs, kv, nk)) > 0.7
    dense_topk, sparse_topk = g, max(1, g // 2)
    os_ = torch.full((bs, kv, nk * g + 4), 7.0, device="cuda")
    oi = torch.full((bs, kv, nk * g + 4), -9, dtype=torch.int64, device="cuda")
    partial_chunk_kivi_qk_dense_sparse_cuda(
        torch.from_numpy(ids).cuda(), torch.from_numpy(dm).cuda(), torch.from_numpy(packed).cuda(),
        to_bf16(mn), to_bf16(mx), to_bf16(q), dense_topk, sparse_topk, g, os_, oi)
    rs, ri = osel.kivi_qk_dense_sparse(ids, dm, packed, mn, mx, q, dense_topk, sparse_topk, g)
    gs, gi = from_torch(os_), from_torch(oi)
    assert np.array_equal(gs[..., :nk * g].view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(gi[..., :nk * g], ri)
    assert np.all(gs[..., nk * g:] == 7.0) and np.all(gi[..., nk * g:] == -9)


@pytest.mark.parametrize("g,dense_topk,sparse_topk,width", [(16, 8, 8, 8), (16, 8, 4, 8), (16, 6, 3, 7),
                                                            (8, 4, 2, 4)])
def test_kivi_qk_compact_output(rng, g, dense_topk, sparse_topk, width):
    """The compact stage-2 output (out_width lanes per chunk) holds the
    oracle's kept lanes at slot * width, leaves the rest of the buffer alone,
    and the global top-k + gather over it picks the same tokens as over the
    full layout whenever no (-1e30, 0) filler can be reached."""
    from zoomkv_revision_amd.kivi import partial_chunk_kivi_qk_dense_sparse_cuda
    from zoomkv_revision_amd.topk import float_topk_gather_concat_3d
    bs, kv, n_chunks, nk, k, sk = 2, 3, 90, 64, 40, 5
    keys = gaussian_bf16(rng, (bs, kv, n_chunks * g, 128), outlier_channels=4)
    mn, mx, _, packed = encode_chunks_ref(keys, g)
    q = gaussian_bf16(rng, (bs, kv, 128))
    ids = rng.integers(0, n_chunks, size=(bs, kv, nk))
    dm = rng.random((bs, kv, nk)) > 0.6
    rs, ri = osel.kivi_qk_dense_sparse(ids, dm, packed, mn, mx, q, dense_topk, sparse_topk, g)
    args = (torch.from_numpy(ids).cuda(), torch.from_numpy(dm).cuda(), torch.from_numpy(packed).cuda(),
            to_bf16(mn), to_bf16(mx), to_bf16(q), dense_topk, sparse_topk, g)
    cs = torch.full((bs, kv, nk * width + 3), 7.0, device="cuda")
    ci = torch.full((bs, kv, nk * width + 3), -9, dtype=torch.int64, device="cuda")
    partial_chunk_kivi_qk_dense_sparse_cuda(*args, cs, ci, out_width=width)
    gs, gi = from_torch(cs), from_torch(ci)
    want_s = rs.reshape(bs, kv, nk, g)[..., :width].reshape(bs, kv, nk * width)
    want_i = ri.reshape(bs, kv, nk, g)[..., :width].reshape(bs, kv, nk * width)
    assert np.array_equal(gs[..., :nk * width].view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(gi[..., :nk * width], want_i)
    assert np.all(gs[..., nk * width:] == 7.0) and np.all(gi[..., nk * width:] == -9)
    # the same final selection as over the full layout (nk * min(keep) >= k)
    assert nk * min(dense_topk, sparse_topk) >= k
    fs = torch.empty(bs, kv, nk * g, device="cuda")
    fi = torch.empty(bs, kv, nk * g, dtype=torch.int64, device="cuda")
    partial_chunk_kivi_qk_dense_sparse_cuda(*args, fs, fi)
    skipped = torch.from_numpy(rng.integers(0, 10 ** 6, size=(bs, kv, sk))).cuda()
    out_full = torch.empty(bs, kv, k + sk, dtype=torch.int64, device="cuda")
    out_compact = torch.empty_like(out_full)
    float_topk_gather_concat_3d(fs, fi, skipped, out_full, k)
    float_topk_gather_concat_3d(cs[..., :nk * width], ci[..., :nk * width], skipped, out_compact, k)
    assert torch.equal(out_full, out_compact)


def test_kivi_qk_compact_rejects_narrow_width(rng):
    from zoomkv_revision_amd._lib import ZkvError
    from zoomkv_revision_amd.kivi import partial_chunk_kivi_qk_dense_sparse_cuda
    g, nk = 16, 4
    keys = gaussian_bf16(rng, (1, 1, 8 * g, 128))
    mn, mx, _, packed = encode_chunks_ref(keys, g)
    q = gaussian_bf16(rng, (1, 1, 128))
    ids = torch.zeros(1, 1, nk, dtype=torch.int64, device="cuda")
    dm = torch.ones(1, 1, nk, dtype=torch.bool, device="cuda")
    o = torch.empty(1, 1, nk * g, device="cuda")
    oi = torch.empty(1, 1, nk * g, dtype=torch.int64, device="cuda")
    with pytest.raises(ZkvError, match="out_width"):
        partial_chunk_kivi_qk_dense_sparse_cuda(ids, dm, torch.from_numpy(packed).cuda(), to_bf16(mn), to_bf16(mx),
                                                to_bf16(q), 8, 8, g, o, oi, out_width=6)


@pytest.mark.parametrize("q_offset", [0, 1])
def test_kivi_qk_unaligned_views(rng, q_offset):
    """Chunk-16 scorer on sliced views: metadata rows from a larger cache
    (nonzero base offset, batch / head strides of the parent), and a query
    row inside a wider store.  q_offset = 0 keeps every query row 16-byte
    aligned (row stride 136 elements), so the host picks the 16-byte load
    path; q_offset = 1 starts each row 2 bytes in (row stride 137), which
    takes the element-wise load path."""
    from zoomkv_revision_amd.kivi import partial_chunk_kivi_qk_dense_sparse_cuda
    g, bs, kv, n_chunks, nk = 16, 3, 2, 50, 41
    keys = gaussian_bf16(rng, (bs, kv, n_chunks * g, 128), outlier_channels=4)
    mn, mx, _, packed = encode_chunks_ref(keys, g)
    q = gaussian_bf16(rng, (bs, kv, 128))
    ids = rng.integers(0, n_chunks, size=(bs, kv, nk))
    dm = rng.random((bs, kv, nk)) > 0.5
    big_mn = torch.zeros(bs, kv + 1, n_chunks + 3, 128, dtype=torch.bfloat16, device="cuda")
    big_mx = torch.zeros_like(big_mn)
    big_mn[:, 1:, 2:2 + n_chunks] = to_bf16(mn)
    big_mx[:, 1:, 2:2 + n_chunks] = to_bf16(mx)
    q_store = torch.zeros(bs, kv, 128 + q_offset + 8, dtype=torch.bfloat16, device="cuda")
    q_store[..., q_offset:q_offset + 128] = to_bf16(q)
    os_ = torch.empty((bs, kv, nk * g), device="cuda")
    oi = torch.empty((bs, kv, nk * g), dtype=torch.int64, device="cuda")
    partial_chunk_kivi_qk_dense_sparse_cuda(
        torch.from_numpy(ids).cuda(), torch.from_numpy(dm).cuda(), torch.from_numpy(packed).cuda(),
        big_mn[:, 1:, 2:2 + n_chunks], big_mx[:, 1:, 2:2 + n_chunks],
        q_store[..., q_offset:q_offset + 128], 16, 5, g, os_, oi)
    rs, ri = osel.kivi_qk_dense_sparse(ids, dm, packed, mn, mx, q, 16, 5, g)
    assert np.array_equal(from_torch(os_).view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(from_torch(oi), ri)


# The reference's own top-k cases (Z/cache_hub/topk/test_float_topk.py:38-149),
# checked here against the exact oracle instead of an overlap count.
@pytest.mark.parametrize("case", ["basic", "k1", "k_near_length", "k_equals_length", "negative",
                                  "mixed_sign", "large_length", "repeated"])
def test_topk_reference_cases(case):
    from zoomkv_revision_amd.topk import float_topk
    g = np.random.default_rng(sorted(["basic", "k1", "k_near_length", "k_equals_length", "negative",
                                      "mixed_sign", "large_length", "repeated"]).index(case))
    shapes = {"basic": (4, 3000, 64), "k1": (8, 500, 1), "k_near_length": (2, 300, 290),
              "k_equals_length": (2, 128, 128), "negative": (4, 1000, 50), "mixed_sign": (4, 2000, 100),
              "large_length": (1, 128 * 1024, 100), "repeated": (1, 1000, 50)}
    B, L, k = shapes[case]
    x = g.standard_normal((B, L)).astype(np.float32)
    if case == "negative":
        x = -g.random((B, L)).astype(np.float32) - 1.0
    elif case == "mixed_sign":
        x *= 100
    elif case == "repeated":
        x[:] = 0
        x[0, :50], x[0, 50:100] = 1.0, 0.5
    got = from_torch(float_topk(torch.from_numpy(x).cuda(), k))
    assert np.array_equal(got, osel.topk_indices(x, k))
    if case == "repeated":
        assert np.all(x[0, got[0]] == 1.0)


# Z/cache_hub/topk/test_float_topk_gather_concat.py:116-128 (same shapes, k, sk and slack)
@pytest.mark.parametrize("bs,kv,L,k,sk,max_sk,seed", [
    (1, 8, 6400, 100, 0, 0, 0), (1, 8, 6400, 100, 12, 12, 1), (8, 8, 6400, 100, 12, 12, 2),
    (8, 8, 6400, 100, 0, 0, 3), (2, 4, 512, 64, 8, 8, 4), (1, 2, 1024, 1, 0, 0, 5),
    (2, 4, 2048, 50, 8, 64, 6)])
def test_gather_concat_reference_cases(bs, kv, L, k, sk, max_sk, seed):
    from zoomkv_revision_amd.topk import float_topk_gather_concat_3d
    g = np.random.default_rng(seed)
    sc = g.standard_normal((bs, kv, L)).astype(np.float32)
    lut = g.integers(0, 1 << 40, size=(bs, kv, L))
    skipped = g.integers(0, 1 << 20, size=(bs, kv, sk))
    out = torch.full((bs, kv, k + max_sk), -5, dtype=torch.int64, device="cuda")
    float_topk_gather_concat_3d(torch.from_numpy(sc).cuda(), torch.from_numpy(lut).cuda(),
                                torch.from_numpy(skipped).cuda(), out, k)
    got = from_torch(out)
    assert np.array_equal(got[..., :k + sk], osel.topk_gather_concat(sc, lut, skipped, k, k + sk))
    assert np.all(got[..., k + sk:] == -5)


@pytest.mark.parametrize("L,k", [(26208, 100), (32768, 512), (32768, 513), (5000, 300), (12000, 1)])
def test_topk_sampled_prefilter_edges(rng, L, k):
    """Rows that steer the sampled prefilter of long rows to each outcome:
    spikes on exactly the 1024 evenly spaced sample positions (fewer keys above
    the threshold than k), integer scores with heavy ties at the threshold, a
    row of one value (more candidates than fit), and a plain row."""
    from zoomkv_revision_amd.topk import float_topk
    x = rng.standard_normal((4, L)).astype(np.float32)
    x[0, (np.arange(1024) * L) // 1024] = 1000.0 + np.arange(1024)
    x[1] = rng.integers(0, 10, L).astype(np.float32)
    x[2] = 3.0
    got = from_torch(float_topk(torch.from_numpy(x).cuda(), k))
    assert np.array_equal(got, osel.topk_indices(x, k))


def test_topk_sentinel_heavy_rows(rng):
    """Rows shaped like the stage-2 scores (half the slots -1e30 per 16), with
    k larger than the number of real values in some rows."""
    from zoomkv_revision_amd.topk import float_topk_3d
    x = (rng.standard_normal((2, 4, 26208)) * 5).astype(np.float32)
    x.reshape(2, 4, -1, 16)[..., 8:] = -1e30
    x[1, 3, 200:] = -1e30                       # only 104 real values, k = 300
    got = from_torch(float_topk_3d(torch.from_numpy(x).cuda(), 300))
    assert np.array_equal(got, osel.topk_indices(x, 300))


@pytest.mark.parametrize("L,k", [(1638, 491), (4096, 1638), (300, 300), (9000, 64), (40000, 100)])
def test_topk_dense_mask_fused_matches_two_ops(rng, L, k):
    """zkv_topk_dense_mask == float_topk_3d then dense_mask_from_topk_cuda."""
    from zoomkv_revision_amd.rerank import dense_mask_from_topk_cuda, topk_dense_mask
    from zoomkv_revision_amd.topk import float_topk_3d
    x = rng.standard_normal((2, 3, L)).astype(np.float32)
    x[1, 1, ::5] = 0.25                                   # ties
    xt = torch.from_numpy(x).cuda()
    ref_idx = float_topk_3d(xt, k)
    ref_mask = torch.ones(2, 3, L, dtype=torch.bool, device="cuda")
    dense_mask_from_topk_cuda(ref_idx, ref_mask)
    mask = torch.ones(2, 3, L, dtype=torch.bool, device="cuda")   # stale contents must be cleared
    idx = topk_dense_mask(xt, k, mask)
    assert torch.equal(idx, ref_idx) and torch.equal(mask, ref_mask)
    assert np.array_equal(from_torch(idx), osel.topk_indices(x, k))


@pytest.mark.parametrize("bs,hq,kv,n_max,n,k,fp16_meta,with_valid", [
    (2, 32, 8, 4096, 4076, 1631, False, True),    # a C5 row: 4076 chunks, top-1631
    (8, 32, 8, 2048, 2048, 128, True, False),      # a C3 row: 2048 fp16 pages, top-128
    (1, 8, 2, 300, 257, 64, False, True),
    (1, 8, 2, 100, 50, 50, False, False),          # k == L
    (1, 8, 2, 100, 30, 40, False, False),          # k > L: every index, then -1
    (2, 16, 4, 130, 129, 1, True, False),
    (1, 4, 1, 4096, 4096, 4000, True, True),       # the longest row
])
def test_quest_topk_fused_equals_two_launches(rng, bs, hq, kv, n_max, n, k, fp16_meta, with_valid):
    """GQA mean + Quest + the row's top-k in one launch (the row's last block
    selects from the device-coherent scores): raw_q and scores bit-identical
    to quest_chunk_score_gqa, indices identical to float_topk_3d on them, and
    to the oracle's; the same over repeated launches on one slots buffer."""
    from zoomkv_revision_amd.quest import quest_chunk_score_gqa, quest_chunk_topk_gqa
    from zoomkv_revision_amd.topk import float_topk_3d
    dt = torch.float16 if fp16_meta else torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(n + k)
    mn = torch.randn(bs, kv, n_max, 128, generator=g, device="cuda").to(dt)
    mx = (mn.float() + torch.rand(bs, kv, n_max, 128, generator=g, device="cuda")).to(dt)
    q = torch.randn(bs, hq, 128, generator=g, device="cuda").to(torch.bfloat16)
    valid = (torch.rand(bs, kv, n_max, generator=g, device="cuda") > 0.05) if with_valid else None
    s1 = torch.empty(bs, kv, n, device="cuda")
    rq1 = torch.empty(bs, kv, 128, dtype=torch.bfloat16, device="cuda")
    quest_chunk_score_gqa(q, kv, mn, mx, s1, n, valid, rq1)
    if k <= n:
        want = float_topk_3d(s1, k)
    else:
        want = torch.cat([torch.arange(n, device="cuda").expand(bs, kv, n),
                          torch.full((bs, kv, k - n), -1, dtype=torch.int64, device="cuda")], -1)
    print(f"[quest topk] bs={bs} kv={kv} n={n} k={k}", flush=True)
    for rep in range(3):
        s2 = torch.full((bs, kv, n), float("nan"), device="cuda")
        rq2 = torch.empty_like(rq1)
        got = quest_chunk_topk_gqa(q, kv, mn, mx, s2, n, valid, rq2, k)
        torch.cuda.synchronize()
        assert torch.equal(rq1.view(torch.int16), rq2.view(torch.int16)), rep
        assert torch.equal(s1.view(torch.int32), s2.view(torch.int32)), rep
        assert torch.equal(got, want), rep
    if k <= n and n <= 300:
        ref = osel.topk_indices(from_torch(s1), k)
        assert np.array_equal(np.sort(from_torch(got), -1), np.sort(ref, -1))


def test_quest_topk_fused_graph_replays():
    """The fused launch captured in a HIP graph: every replay, with eager
    launches on other inputs (other epochs, the same slots buffer) in
    between, equals the eager result."""
    from zoomkv_revision_amd.quest import quest_chunk_topk_gqa
    bs, hq, kv, n, k = 2, 32, 8, 2048, 128
    g = torch.Generator(device="cuda").manual_seed(3)
    ins = []
    for _ in range(2):
        mn = torch.randn(bs, kv, n, 128, generator=g, device="cuda").to(torch.float16)
        mx = (mn.float() + torch.rand(bs, kv, n, 128, generator=g, device="cuda")).to(torch.float16)
        q = torch.randn(bs, hq, 128, generator=g, device="cuda").to(torch.bfloat16)
        ins.append((q, mn, mx))
    bufs = [(torch.empty(bs, kv, n, device="cuda"), torch.empty(bs, kv, 128, dtype=torch.bfloat16, device="cuda"),
             torch.empty(bs, kv, k, dtype=torch.int64, device="cuda")) for _ in range(2)]
    run = lambda i: quest_chunk_topk_gqa(ins[i][0], kv, ins[i][1], ins[i][2], bufs[i][0], n, None, bufs[i][1], k,
                                         bufs[i][2])
    eager = []
    for i in range(2):
        run(i)
        eager.append(bufs[i][2].clone())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(0)
    for rep in range(4):
        bufs[0][2].fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bufs[0][2], eager[0]), f"replay {rep}"
        run(1)
        torch.cuda.synchronize()
        assert torch.equal(bufs[1][2], eager[1]), f"eager after replay {rep}"
