"""The in-launch split merge against the separate merge kernel.

With more than one context split, the workgroup that completes a (b, kv)
merges the splits' partials inside the attention launch (the default);
ZKV_SPLIT_MERGE=kernel runs the separate merge kernel instead.  Both merge in
split order with the same arithmetic, so outputs and LSEs must be
bit-identical -- whatever the workspace held before (the arrival slots carry
a per-launch epoch and need no zeroing), over repeated launches that reuse
one workspace with different split counts, and whichever split arrives last.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _garbage_workspace(nbytes, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=g)


def _bits(t):
    t = t.detach()
    return (t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)).cpu().numpy()


def _same_bits(a, b):
    if isinstance(a, tuple):
        return all(_same_bits(x, y) for x, y in zip(a, b))
    return np.array_equal(_bits(a), _bits(b))


def _both(monkeypatch, fn):
    """fn() with the merge kernel, then with the in-launch merge (device-
    coherent partials, the default); the in-launch merge ordered by
    agent-scope fences (ZKV_SPLIT_MERGE=fence) must give the same bits."""
    monkeypatch.setenv("ZKV_SPLIT_MERGE", "kernel")
    ref = fn()
    torch.cuda.synchronize()
    monkeypatch.setenv("ZKV_SPLIT_MERGE", "fence")
    fenced = fn()
    torch.cuda.synchronize()
    fenced = tuple(t.clone() for t in fenced) if isinstance(fenced, tuple) else fenced.clone()
    monkeypatch.delenv("ZKV_SPLIT_MERGE")
    got = fn()
    torch.cuda.synchronize()
    assert _same_bits(fenced, got), "fence-ordered merge differs from the device-coherent one"
    return ref, got


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_dense_in_launch_merge_bit_exact(monkeypatch, out_dtype):
    from zoomkv_revision_amd import kivi, synthetic
    dev = torch.device("cuda:0")
    bs, hq, kv, ng, r = 3, 8, 2, 40, 50
    cache = synthetic.c2_cache(7, bs, kv, ng, r, dev)
    q = synthetic.c2_query(bs, hq, dev, seed=3)
    ws = _garbage_workspace(kivi.lib().zkv_kivi4_attention_workspace_size(bs, hq, kv, ng, r, 8), 11)
    print(f"[split merge] dense bs={bs} hq={hq} kv={kv} groups={ng} res={r} out={out_dtype}", flush=True)
    for rep in range(2):
        for n_splits in (2, 3, 5, 8, 0):
            ref, got = _both(monkeypatch, lambda: kivi.kivi4_decode_attention(
                q, cache, ng, r, out_dtype=out_dtype, n_splits=n_splits, workspace=ws))
            assert np.isfinite(ref.float().cpu().numpy()).all()
            assert np.array_equal(_bits(ref), _bits(got)), f"rep {rep} n_splits {n_splits}"


def test_dense_in_launch_merge_matches_single_split(monkeypatch):
    """The merged output stays within the splits' fp16 rounding of one split."""
    from zoomkv_revision_amd import kivi, synthetic
    dev = torch.device("cuda:0")
    bs, hq, kv, ng, r = 2, 16, 4, 64, 128
    cache = synthetic.c2_cache(21, bs, kv, ng, r, dev)
    q = synthetic.c2_query(bs, hq, dev, seed=5)
    one = kivi.kivi4_decode_attention(q, cache, ng, r, out_dtype=torch.float32, n_splits=1)
    for n_splits in (2, 4, 7):
        got = kivi.kivi4_decode_attention(q, cache, ng, r, out_dtype=torch.float32, n_splits=n_splits)
        assert (got - one).abs().max().item() <= 1e-3, n_splits


def test_sparse_in_launch_merge_bit_exact(monkeypatch):
    from zoomkv_revision_amd import kivi, synthetic
    dev = torch.device("cuda:0")
    bs, hq, kv = 2, 8, 2
    w = synthetic.c3_workload(17, bs, hq, kv, 4096, 40, dev)
    pages = w["planted"]
    print(f"[split merge] sparse bs={bs} pages={pages.shape[-1]}", flush=True)
    for n_splits in (2, 4, 3):
        ref, got = _both(monkeypatch, lambda: kivi.kivi4_sparse_attention(
            w["q"], w["cache"], pages, out_dtype=torch.float32, n_splits=n_splits))
        assert np.array_equal(_bits(ref), _bits(got)), n_splits


def test_bf16_in_launch_merge_bit_exact_with_lse(monkeypatch):
    from zoomkv_revision_amd import attention
    g = torch.Generator(device="cuda").manual_seed(8)
    bs, hq, kv, n = 2, 8, 2, 700
    q = torch.randn(bs, 1, hq, 128, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(bs, n, kv, 128, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(bs, n, kv, 128, device="cuda", generator=g).to(torch.bfloat16)
    print(f"[split merge] bf16 bs={bs} n={n}", flush=True)
    for n_splits in (2, 3, 6):
        (ro, rl), (go, gl) = _both(monkeypatch, lambda: attention.flash_attn_with_kvcache_compat(
            q, k, v, return_softmax_lse=True, n_splits=n_splits))
        assert np.array_equal(_bits(ro), _bits(go)), n_splits
        assert np.array_equal(_bits(rl), _bits(gl)), n_splits


def test_gather_in_launch_merge_bit_exact(monkeypatch):
    from zoomkv_revision_amd import attention
    g = torch.Generator(device="cuda").manual_seed(9)
    bs, hq, kv, rows = 2, 8, 2, 900
    q = torch.randn(bs, 1, hq, 128, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(bs, kv, rows, 128, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(bs, kv, rows, 128, device="cuda", generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 600, (bs, kv, 300), device="cuda", generator=g)
    for n_splits in (2, 5):
        (ro, rl), (go, gl) = _both(monkeypatch, lambda: attention.gather_attention(
            q, k, v, idx, tail_start=600, tail_len=300, return_softmax_lse=True, n_splits=n_splits))
        assert np.array_equal(_bits(ro), _bits(go)), n_splits
        assert np.array_equal(_bits(rl), _bits(gl)), n_splits


def test_in_launch_merge_graph_replays(monkeypatch):
    """A captured launch keeps its epoch: every replay must still merge (the
    last arrival resets the count), with eager launches on the same workspace
    -- other epochs, other split counts -- between the replays."""
    from zoomkv_revision_amd import kivi, synthetic
    monkeypatch.delenv("ZKV_SPLIT_MERGE", raising=False)
    dev = torch.device("cuda:0")
    bs, hq, kv, ng, r = 2, 8, 2, 48, 64
    caches = [synthetic.c2_cache(31 + i, bs, kv, ng, r, dev) for i in range(2)]
    q = synthetic.c2_query(bs, hq, dev, seed=4)
    ws = _garbage_workspace(kivi.lib().zkv_kivi4_attention_workspace_size(bs, hq, kv, ng, r, 6), 12)
    outs = [torch.empty(bs, hq, 128, dtype=torch.float32, device=dev) for _ in range(2)]
    eager = [kivi.kivi4_decode_attention(q, c, ng, r, out=o, out_dtype=torch.float32, n_splits=3, workspace=ws).clone()
             for c, o in zip(caches, outs)]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kivi.kivi4_decode_attention(q, caches[0], ng, r, out=outs[0], out_dtype=torch.float32, n_splits=3, workspace=ws)
    for rep in range(4):
        outs[0].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs[0].view(torch.int32), eager[0].view(torch.int32)), f"replay {rep}"
        got = kivi.kivi4_decode_attention(q, caches[1], ng, r, out=outs[1], out_dtype=torch.float32,
                                          n_splits=3 + rep % 2, workspace=ws)
        torch.cuda.synchronize()
        if rep % 2 == 0:
            assert torch.equal(got.view(torch.int32), eager[1].view(torch.int32)), f"eager after replay {rep}"
        else:
            assert (got - eager[1]).abs().max().item() <= 1e-3


@pytest.mark.parametrize("hq,kv,n_splits", [(16, 1, 12), (32, 8, 20), (8, 2, 9)])
def test_in_launch_merge_many_splits(monkeypatch, hq, kv, n_splits):
    """More than 8 splits (the merge's unbatched loop) and 16 query heads per
    KV head: the in-launch merge equals the merge kernel bit for bit."""
    from zoomkv_revision_amd import kivi, synthetic
    dev = torch.device("cuda:0")
    bs, ng, r = 2, 200, 70
    cache = synthetic.c2_cache(41, bs, kv, ng, r, dev)
    q = synthetic.c2_query(bs, hq, dev, seed=6)
    ws = _garbage_workspace(kivi.lib().zkv_kivi4_attention_workspace_size(bs, hq, kv, ng, r, n_splits), 13)
    print(f"[split merge] many splits hq={hq} kv={kv} n_splits={n_splits}", flush=True)
    _, used = kivi.kivi4_attention_partial(q, cache, ng, r, n_splits=n_splits, workspace=ws)
    assert used > 8
    ref, got = _both(monkeypatch, lambda: kivi.kivi4_decode_attention(
        q, cache, ng, r, out_dtype=torch.float32, n_splits=n_splits, workspace=ws))
    assert np.isfinite(ref.cpu().numpy()).all()
    assert np.array_equal(_bits(ref), _bits(got))


def test_workspace_without_arrival_slots_is_rejected():
    """A workspace sized for the split partials only (no arrival slots) is
    too small for a merging launch: the call fails with ZKV_ESPACE and runs
    nothing."""
    from zoomkv_revision_amd import kivi, synthetic
    from zoomkv_revision_amd._lib import ZkvError
    dev = torch.device("cuda:0")
    bs, hq, kv, ng, r = 2, 8, 2, 40, 32
    cache = synthetic.c2_cache(51, bs, kv, ng, r, dev)
    q = synthetic.c2_query(bs, hq, dev, seed=7)
    need = kivi.lib().zkv_kivi4_attention_workspace_size(bs, hq, kv, ng, r, 4)
    partials_only = bs * hq * 4 * (128 + 2) * 4
    assert need == partials_only + bs * kv * 8
    ws = torch.zeros(partials_only, dtype=torch.uint8, device=dev)
    with pytest.raises(ZkvError, match="workspace"):
        kivi.kivi4_decode_attention(q, cache, ng, r, n_splits=4, workspace=ws)


def test_in_launch_merge_ignores_small_integer_slots(monkeypatch):
    """A reused workspace whose arrival slots hold small int64 values of the
    form (k << 8) | c (token indices, counts: what an allocator hands back
    after other ops) must never read as a live launch's slot.  Epochs carry
    bit 55 and a random per-process base, so with k over a wide range and
    every count c below the split count, a few hundred launches all equal the
    separate merge kernel bit for bit."""
    from zoomkv_revision_amd import kivi, synthetic
    dev = torch.device("cuda:0")
    bs, hq, kv, ng, r, n_splits = 3, 8, 2, 40, 50, 4
    cache = synthetic.c2_cache(61, bs, kv, ng, r, dev)
    q = synthetic.c2_query(bs, hq, dev, seed=9)
    need = kivi.lib().zkv_kivi4_attention_workspace_size(bs, hq, kv, ng, r, n_splits)
    slot0 = need - bs * kv * 8
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    slots = ws[slot0:].view(torch.int64)
    monkeypatch.setenv("ZKV_SPLIT_MERGE", "kernel")
    ref = kivi.kivi4_decode_attention(q, cache, ng, r, out_dtype=torch.float32, n_splits=n_splits,
                                      workspace=ws).clone()
    monkeypatch.delenv("ZKV_SPLIT_MERGE")
    out = torch.empty_like(ref)
    n_slots = bs * kv
    print(f"[split merge] small-integer slots: 300 launches, {n_slots} slots", flush=True)
    for rep in range(300):
        k = torch.arange(rep * n_slots, (rep + 1) * n_slots, dtype=torch.int64, device=dev)
        slots.copy_((k << 8) | (k % n_splits))
        out.zero_()
        kivi.kivi4_decode_attention(q, cache, ng, r, out=out, out_dtype=torch.float32, n_splits=n_splits,
                                    workspace=ws)
        if rep % 50 == 49:
            torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"launch {rep}"
