"""GPU: the C5 decode step over the real polar_cache (small model, 4096-token
context, sparse selection on, one flush inside the run)."""
import pytest
import torch

from zoomkv_revision_amd import decode_step as ds

pytestmark = pytest.mark.gpu


def test_decode_steps_through_polar_cache_with_a_flush(monkeypatch):
    for k, v in ds.PRODUCTION_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.delenv("POLAR_FORCE_CAND_TOKENS", raising=False)
    geo = ds.Qwen3Geometry(layers=2, hidden=256, heads=32, kv_heads=8, head_dim=128, ffn=512, vocab=1000)
    dev = torch.device("cuda:0")
    batch, context, interval, steps = 2, 4096, 64, 70
    model = ds.RandomQwen3(geo, dev, seed=42, max_position=8192)
    cache = ds.build_cache(geo, batch, context, steps + 8, interval, 2048, dev)
    ds.fill_cache(cache, geo, batch, context, 43, dev)
    retrieval0 = int(cache.cpu_valid_end[0])
    gen = torch.Generator(device=dev).manual_seed(42)
    tok = torch.randint(0, geo.vocab, (batch,), generator=gen, device=dev)
    seen = []
    for _ in range(steps):
        logits = model.decode_step(tok, cache)
        tok = ds.sample_next_token(logits, 0.6, 0.95, 20, generator=gen)
        seen.append(tok)
    torch.cuda.synchronize()
    assert cache.context == context + steps
    assert int(cache.cpu_valid_end[0]) == retrieval0 + interval          # one flush of 64 tokens
    assert cache._last_topk_indices is not None                          # the sparse path ran
    assert torch.isfinite(logits).all()
    toks = torch.stack(seen)
    assert ((toks >= 0) & (toks < geo.vocab)).all()
    b = ds.attention_path_bytes(cache, 0)
    assert b["total"] > b["quest"] > 0
