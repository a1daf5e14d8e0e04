"""The decode path captured in a HIP graph (the reference built its fused
top-k to stay graph-friendly, S:361-367): polar_cache.compute of every layer,
and a whole decode step (36-layer-style model pass up to the logits; the
sampler's tie check reads the host and stays outside), in both storage modes
(bf16 retrieval zone and the 4-bit K + V zone).

A graph is captured at the cache's current position and replayed several
times, with eager work on other inputs and synchronisations between the
replays; every replay equals the eager result bit for bit (the kernels are
deterministic: fixed split plans, fixed merge orders).  A captured step
re-runs the same token at the same position: the host bookkeeping advanced
once, during the capture, and the K / V append rewrites the same row with the
same values on every replay.

Geometry: 3 layers of 32 / 8 heads of 128, hidden 1024, FFN 2048, vocabulary
8192 (random-init bf16), batch 2, an 8192-token prompt (above the 2048-token
full-attention threshold, so the sparse selection runs), the production
cache knobs."""
import pytest
import torch

pytestmark = pytest.mark.gpu

BATCH, CONTEXT, INTERVAL, THRESHOLD = 2, 8192, 512, 2048


@pytest.fixture(scope="module", params=["bf16", "kivi4"])
def setup(request):
    from zoomkv_revision_amd import decode_step as ds
    mp = pytest.MonkeyPatch()
    for k, v in ds.PRODUCTION_ENV.items():
        mp.setenv(k, v)
    mp.delenv("POLAR_FORCE_CAND_TOKENS", raising=False)
    geo = ds.Qwen3Geometry(layers=3, hidden=1024, ffn=2048, vocab=8192)
    dev = torch.device("cuda:0")
    model = ds.RandomQwen3(geo, dev, seed=7, max_position=CONTEXT + 64)
    cache = ds.build_cache(geo, BATCH, CONTEXT, 16, INTERVAL, THRESHOLD, dev, kv_format=request.param)
    ds.fill_cache(cache, geo, BATCH, CONTEXT, 8, dev)
    torch.cuda.synchronize()
    print(f"[graph] storage {request.param}: cache filled", flush=True)
    yield {"ds": ds, "geo": geo, "model": model, "cache": cache, "dev": dev}
    mp.undo()
    del cache, model
    torch.cuda.empty_cache()


def _host_state(cache):
    return list(cache.current_seq_len), cache.context, cache._decode_step_counter


def _set_host_state(cache, st):
    cache.current_seq_len[:] = st[0]
    cache.context, cache._decode_step_counter = st[1], st[2]


def test_cache_compute_graph_replays_match_eager(setup):
    geo, cache, dev = setup["geo"], setup["cache"], setup["dev"]
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    qs = [torch.randn(BATCH, 1, geo.heads, geo.head_dim, generator=g, device=dev).to(torch.bfloat16)
          for _ in range(2 * geo.layers)]

    def attend(qset):
        return [cache.compute(q, ldx) for ldx, q in enumerate(qset)]

    eager = [t.clone() for t in attend(qs[:geo.layers])]
    other = [t.clone() for t in attend(qs[geo.layers:])]
    assert cache._last_topk_indices is not None      # the sparse selection ran
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = attend(qs[:geo.layers])
    for rep in range(4):
        for t in outs:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for ldx, (a, b) in enumerate(zip(outs, eager)):
            assert torch.equal(a, b), f"replay {rep}, layer {ldx}"
        # eager work on other queries between replays
        got = attend(qs[geo.layers:])
        torch.cuda.synchronize()
        for a, b in zip(got, other):
            assert torch.equal(a, b)
    print(f"[graph] compute of {geo.layers} layers: 4 replays equal eager", flush=True)


def test_decode_step_graph_replays_match_eager(setup):
    geo, model, cache, dev = setup["geo"], setup["model"], setup["cache"], setup["dev"]
    tok = torch.tensor([5, 4000], device=dev)
    tok2 = torch.tensor([17, 9], device=dev)
    st = _host_state(cache)
    logits = model.decode_step(tok, cache).clone()
    torch.cuda.synchronize()
    _set_host_state(cache, st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        logits_g = model.decode_step(tok, cache)
    after = _host_state(cache)
    assert after[1] == st[1] + 1                      # the capture ran the step's bookkeeping once
    for rep in range(3):
        logits_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits_g, logits), f"replay {rep}"
        # an eager step of another token at the same position, then the
        # replayed token's K / V row is rewritten by the next replay
        _set_host_state(cache, st)
        other = model.decode_step(tok2, cache)
        torch.cuda.synchronize()
        assert torch.isfinite(other).all()
        _set_host_state(cache, after)
    print(f"[graph] decode step: 3 replays equal eager (logits max {logits.abs().max().item():.3f})", flush=True)
