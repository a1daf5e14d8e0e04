"""GPU parity of the C3 path: fp16 Quest page metadata (bit-exact), page-sparse
4-bit decode attention (within 2e-3 of the oracle) and the planted-page
select -> attend pipeline (selection equals the planted set)."""
import numpy as np
import pytest
import torch

from oracle import kivi as okivi
from oracle import select as osel
from tests.helpers import from_torch, gaussian_bf16, to_bf16

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _bits16(t):
    return from_torch(t.view(torch.int16)).view(np.uint16)


def test_page_minmax_f16_bit_exact(rng):
    from zoomkv_revision_amd.quest import page_minmax_f16
    k = gaussian_bf16(rng, (2, 3, 40 * 16 + 5, 128), outlier_channels=3)
    k[0, 1, 17, 9] = 2e5          # above fp16 max: max rounds to +inf, min of other pages unaffected
    k[1, 2, 100, 4] = -7e-9       # below fp16 subnormals
    k[1, 0, 33, 0] = 3.1e-6       # fp16 subnormal range: inexact, directed rounding matters
    kt = to_bf16(np.ascontiguousarray(np.swapaxes(k, 1, 2))).transpose(1, 2)   # strided tokens
    mn, mx = page_minmax_f16(kt, 16)
    rmn, rmx = osel.page_minmax_f16(k, 16)
    assert np.array_equal(_bits16(mn), rmn) and np.array_equal(_bits16(mx), rmx)


def _pack(rng, bs, kv, ng):
    from zoomkv_revision_amd import kivi
    k = gaussian_bf16(rng, (bs, kv, ng * 32, 128), outlier_channels=1)
    v = gaussian_bf16(rng, (bs, kv, ng * 32, 128))      # outlier channels are a K phenomenon
    cache = kivi.Kivi4Cache.allocate(bs, kv, ng, 128)
    kivi.kivi4_pack(to_bf16(k), to_bf16(v), cache, 0)
    return okivi.quantize_kivi4(k, v), cache


def _pages(rng, kind, bs, kv, ng, n_sel):
    n_pages = 2 * ng
    if kind == "sorted":
        return np.sort(np.stack([[rng.choice(n_pages, n_sel, replace=False) for _ in range(kv)]
                                 for _ in range(bs)]), -1)
    if kind == "unsorted":
        return np.stack([[rng.choice(n_pages, n_sel, replace=False) for _ in range(kv)] for _ in range(bs)])
    if kind == "pairs":          # whole groups: every tile takes both halves
        g = np.sort(np.stack([[rng.choice(ng, n_sel // 2, replace=False) for _ in range(kv)]
                              for _ in range(bs)]), -1)
        return np.stack([2 * g, 2 * g + 1], -1).reshape(bs, kv, -1)
    if kind == "messy":          # duplicates, out-of-range ids, unsorted
        p = rng.integers(-3, n_pages + 3, size=(bs, kv, n_sel))
        p[..., 1] = p[..., 0]
        return p
    if kind == "all":
        return np.broadcast_to(np.arange(n_pages), (bs, kv, n_pages)).copy()
    raise ValueError(kind)


@pytest.mark.parametrize("bs,hq,kv,ng,res,n_sel,kind,splits", [
    (2, 32, 8, 40, 0, 24, "sorted", 0),
    (2, 32, 8, 40, 50, 24, "unsorted", 0),
    (1, 8, 2, 30, 0, 20, "pairs", 0),
    (2, 8, 2, 30, 17, 40, "messy", 0),
    (1, 8, 2, 12, 128, 24, "all", 0),
    (1, 8, 2, 12, 0, 1, "sorted", 0),
    (2, 8, 2, 20, 0, 16, "sorted", 1),
    (1, 8, 2, 600, 0, 1100, "sorted", 1),   # > 512 tiles: the planner splits anyway
    (1, 16, 1, 30, 10, 21, "messy", 0),     # 16 query heads per KV head
    (2, 16, 2, 30, 10, 21, "unsorted", 0),  # 8 query heads per KV head
])
def test_sparse_attention_matches_oracle(rng, bs, hq, kv, ng, res, n_sel, kind, splits):
    from zoomkv_revision_amd import kivi
    ref_cache, cache = _pack(rng, bs, kv, ng)
    kr = gaussian_bf16(rng, (bs, kv, 128, 128))
    vr = gaussian_bf16(rng, (bs, kv, 128, 128))
    cache.k_res.copy_(to_bf16(kr))
    cache.v_res.copy_(to_bf16(vr))
    q = gaussian_bf16(rng, (bs, hq, 128))
    pages = _pages(rng, kind, bs, kv, ng, n_sel)
    pt = torch.from_numpy(pages).cuda()
    got = from_torch(kivi.kivi4_sparse_attention(to_bf16(q), cache, pt, ng, res, out_dtype=torch.float32,
                                                 n_splits=splits))
    ref = okivi.kivi4_sparse_attention(q, ref_cache, ng, kr, vr, res, pages, 1 / np.sqrt(128))
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs err {err}"
    if kind == "all":
        dense = from_torch(kivi.kivi4_decode_attention(to_bf16(q), cache, ng, res, out_dtype=torch.float32))
        assert np.abs(got - dense).max() <= 1e-3


def test_sparse_attention_empty_list_and_residual_only(rng):
    from zoomkv_revision_amd import kivi
    ref_cache, cache = _pack(rng, 1, 2, 4)
    kr = gaussian_bf16(rng, (1, 2, 128, 128))
    vr = gaussian_bf16(rng, (1, 2, 128, 128))
    cache.k_res.copy_(to_bf16(kr))
    cache.v_res.copy_(to_bf16(vr))
    q = gaussian_bf16(rng, (1, 8, 128))
    none = torch.full((1, 2, 3), -1, dtype=torch.int64, device="cuda")
    got = from_torch(kivi.kivi4_sparse_attention(to_bf16(q), cache, none, 4, 33, out_dtype=torch.float32))
    ref = okivi.kivi4_sparse_attention(q, ref_cache, 4, kr, vr, 33, -np.ones((1, 2, 3), int), 1 / np.sqrt(128))
    assert np.abs(got - ref).max() <= ATOL
    # nothing to attend: zeros (no NaN)
    z = from_torch(kivi.kivi4_sparse_attention(to_bf16(q), cache, none, 4, 0, out_dtype=torch.float32))
    assert np.all(z == 0)


def test_c3_planted_pipeline_small(rng):
    """GQA mean -> Quest over fp16 page metadata -> top-k pages -> sparse
    attention, at a reduced C3 shape; the selection must be the planted set."""
    from zoomkv_revision_amd import kivi, synthetic
    from zoomkv_revision_amd.quest import quest_chunk_score
    from zoomkv_revision_amd.topk import float_topk_3d
    w = synthetic.c3_workload(7, 2, 32, 8, 4096, 24, "cuda", keep_keys=True)
    bs, kv, n_pages = 2, 8, w["n_pages"]
    scores = torch.empty(bs, kv, n_pages, device="cuda")
    quest_chunk_score(w["raw_q"], w["page_min"], w["page_max"], scores, n_pages)
    sel = float_topk_3d(scores, 24)
    assert torch.equal(sel, w["planted"])
    # scores: bit-exact against the oracle on the same metadata
    f16 = lambda t: from_torch(t).view(np.float16).astype(np.float32)   # from_torch gives fp16 bits
    ref_sc = osel.quest_chunk_score(from_torch(w["raw_q"]), f16(w["page_min"]), f16(w["page_max"]), n_pages)
    assert np.array_equal(from_torch(scores).view(np.uint32), ref_sc.view(np.uint32))
    out = from_torch(kivi.kivi4_sparse_attention(w["q"], w["cache"], sel, out_dtype=torch.float32))
    ref_cache = okivi.quantize_kivi4(from_torch(w["k"]), from_torch(w["v"]))
    z = np.zeros((bs, kv, 0, 128), np.float32)
    ref = okivi.kivi4_sparse_attention(from_torch(w["q"]), ref_cache, 128, z, z, 0, from_torch(sel),
                                       1 / np.sqrt(128))
    assert np.abs(out - ref).max() <= ATOL


def test_c3_full_size_selection_is_the_planted_set():
    """BASELINE config 3 shape: batch 8, 32/8 heads, 32768 tokens = 2048 pages,
    top-128 pages."""
    from zoomkv_revision_amd import synthetic
    from zoomkv_revision_amd.quest import quest_chunk_score
    from zoomkv_revision_amd.topk import float_topk_3d
    w = synthetic.c3_workload(42, 8, 32, 8, 32768, 128, "cuda")
    scores = torch.empty(8, 8, 2048, device="cuda")
    quest_chunk_score(w["raw_q"], w["page_min"], w["page_max"], scores, 2048)
    assert torch.equal(float_topk_3d(scores, 128), w["planted"])
    # margin of the planted construction: >= 5% between the sets
    s = scores.sort(dim=-1, descending=True).values
    assert bool((s[..., 127] >= 1.05 * s[..., 128]).all())


def test_c3_pipeline_graph_replays_match_eager():
    """The C3 step (GQA mean + Quest, top-k pages, page-sparse attention)
    captured in a HIP graph: every replay, with eager work on other inputs and
    synchronisations in between, equals the eager result (no library call in
    the chain records a memset)."""
    from zoomkv_revision_amd import kivi, synthetic
    from zoomkv_revision_amd.quest import quest_chunk_score_gqa
    from zoomkv_revision_amd.topk import float_topk_3d
    bs, hq, kv, n_tok, n_sel = 2, 32, 8, 4096, 24
    ws = [synthetic.c3_workload(11 + i, bs, hq, kv, n_tok, n_sel, "cuda") for i in range(2)]
    n_pages = ws[0]["n_pages"]

    def step(w, scores, raw_q, out):
        quest_chunk_score_gqa(w["q"], kv, w["page_min"], w["page_max"], scores, n_pages, None, raw_q)
        sel = float_topk_3d(scores, n_sel)
        kivi.kivi4_sparse_attention(w["q"], w["cache"], sel, out=out)
        return sel

    bufs = [(torch.empty(bs, kv, n_pages, device="cuda"), torch.empty(bs, kv, 128, dtype=torch.bfloat16, device="cuda"),
             torch.empty(bs, hq, 128, dtype=torch.bfloat16, device="cuda")) for _ in ws]
    eager = []
    for w, b in zip(ws, bufs):
        sel = step(w, *b)
        eager.append((sel.clone(), b[2].clone()))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sel_g = step(ws[0], *bufs[0])
    for rep in range(4):
        bufs[0][2].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(sel_g, eager[0][0]), f"replay {rep}: selection"
        assert torch.equal(bufs[0][2], eager[0][1]), f"replay {rep}: attention output"
        assert torch.equal(sel_g, ws[0]["planted"])
        # eager work on the other workload between replays
        sel1 = step(ws[1], *bufs[1])
        torch.cuda.synchronize()
        assert torch.equal(sel1, eager[1][0]) and torch.equal(bufs[1][2], eager[1][1])


def test_sparse_attention_zero_pages_is_residual_only(rng):
    """An empty page list (n_sel = 0) attends the residual window only."""
    from zoomkv_revision_amd import kivi
    ref_cache, cache = _pack(rng, 1, 2, 6)
    kr = gaussian_bf16(rng, (1, 2, 128, 128))
    vr = gaussian_bf16(rng, (1, 2, 128, 128))
    cache.k_res.copy_(to_bf16(kr))
    cache.v_res.copy_(to_bf16(vr))
    q = gaussian_bf16(rng, (1, 8, 128))
    empty = torch.empty(1, 2, 0, dtype=torch.int64, device="cuda")
    got = from_torch(kivi.kivi4_sparse_attention(to_bf16(q), cache, empty, 6, 40, out_dtype=torch.float32))
    ref = okivi.kivi4_sparse_attention(q, ref_cache, 6, kr, vr, 40, np.zeros((1, 2, 0), int), 1 / np.sqrt(128))
    assert np.abs(got - ref).max() <= ATOL


def _oracle_records(cache, b):
    """The GPU cache's Format Q records of sequence b as the oracle's arrays."""
    f16 = lambda t: t.cpu().view(torch.int16).numpy().view(np.uint16)
    return okivi.Kivi4Cache(cache.k_codes[b:b + 1].cpu().numpy(), f16(cache.k_meta[b:b + 1]),
                            cache.v_codes[b:b + 1].cpu().numpy(), f16(cache.v_meta[b:b + 1]))


def test_c3_full_shape_sparse_attention_matches_oracle():
    """BASELINE config 3 at its own shape (batch 8, 32 / 8 heads, 32768 tokens,
    the 128 planted pages of each (b, kv)), with the bench's automatic plan:
    4 context splits merged inside the launch.  Outputs of sequences 0 and 7
    (all 32 query heads) within 2e-3 of the float64 oracle over the cache's
    records, and their natural-log LSEs within 1e-5 relative (a dropped or
    repeated tile moves the LSE by ~1e-4 relative here)."""
    from zoomkv_revision_amd import kivi, synthetic
    bs, hq, kv, n_tok, n_sel = 8, 32, 8, 32768, 128
    w = synthetic.c3_workload(42, bs, hq, kv, n_tok, n_sel, "cuda")
    need = kivi.lib().zkv_kivi4_sparse_attention_workspace_size(bs, hq, kv, n_sel, 0, 0)
    splits = (need - bs * kv * 8) // (bs * hq * 130 * 4)
    assert splits == 4 and need == bs * hq * splits * 130 * 4 + bs * kv * 8
    out, lse = kivi.kivi4_sparse_attention(w["q"], w["cache"], w["planted"], out_dtype=torch.float32,
                                           return_lse=True)
    out, lse = from_torch(out), from_torch(lse)
    qn, pages = from_torch(w["q"]), from_torch(w["planted"])
    z = np.zeros((1, kv, 0, 128), np.float32)
    for b in (0, 7):
        ref, ref_lse = okivi.kivi4_sparse_attention(qn[b:b + 1], _oracle_records(w["cache"], b), n_tok // 32, z, z,
                                                    0, pages[b:b + 1], 1 / np.sqrt(128), return_lse=True)
        err = np.abs(out[b:b + 1] - ref).max()
        lerr = np.abs(lse[b:b + 1] / ref_lse - 1).max()
        print(f"[c3 full] sequence {b}: max abs err {err:.3e}, LSE rel err {lerr:.3e}", flush=True)
        assert err <= ATOL, f"sequence {b}: max abs err {err}"
        assert lerr <= 1e-5, f"sequence {b}: LSE rel err {lerr}"


def test_c3_plans_match_the_calls():
    """QuestTopkPlan and SparseAttentionPlan (checks once, one C-ABI call per
    run) give the calls' bits on the buffers' current contents: the query is
    rewritten in place between runs."""
    from zoomkv_revision_amd import kivi, synthetic
    from zoomkv_revision_amd.quest import QuestTopkPlan, quest_chunk_topk_gqa
    bs, hq, kv, n_tok, n_sel = 2, 16, 4, 4096, 24
    ws = [synthetic.c3_workload(300 + i, bs, hq, kv, n_tok, n_sel, torch.device("cuda")) for i in range(2)]
    n_pages = ws[0]["n_pages"]
    scores = torch.empty(bs, kv, n_pages, device="cuda")
    raw_q = torch.empty(bs, kv, 128, dtype=torch.bfloat16, device="cuda")
    sel = torch.empty(bs, kv, n_sel, dtype=torch.int64, device="cuda")
    out = torch.empty(bs, hq, 128, dtype=torch.float32, device="cuda")
    q_buf = ws[0]["q"].clone()
    w = ws[0]
    qplan = QuestTopkPlan(q_buf, kv, w["page_min"], w["page_max"], scores, n_pages, None, raw_q, n_sel, sel)
    splan = kivi.SparseAttentionPlan(q_buf, w["cache"], sel, out=out, out_dtype=torch.float32, return_lse=True)
    for src in (ws[0]["q"], ws[1]["q"]):
        q_buf.copy_(src)
        got_sel = qplan.run().clone()
        got_out, got_lse = splan.run()
        want_sel = quest_chunk_topk_gqa(src, kv, w["page_min"], w["page_max"], torch.empty_like(scores), n_pages,
                                        None, torch.empty_like(raw_q), n_sel)
        want_out, want_lse = kivi.kivi4_sparse_attention(src, w["cache"], want_sel, out_dtype=torch.float32,
                                                         return_lse=True)
        assert torch.equal(got_sel, want_sel)
        assert torch.equal(got_out.view(torch.int32), want_out.view(torch.int32))
        assert torch.equal(got_lse.view(torch.int32), want_lse.view(torch.int32))


def test_sparse_plan_rejects_a_strided_page_list(rng):
    from zoomkv_revision_amd import kivi
    bs, hq, kv = 1, 8, 2
    cache = kivi.Kivi4Cache.allocate(bs, kv, 4, 32)
    q = to_bf16(gaussian_bf16(rng, (bs, hq, 128)))
    pages = torch.zeros(bs, kv, 8, 2, dtype=torch.int64, device="cuda")[..., 0]   # last-dim stride 2
    with pytest.raises(ValueError, match="in place"):
        kivi.SparseAttentionPlan(q, cache, pages, 4, 0)
