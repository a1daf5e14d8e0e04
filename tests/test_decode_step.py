"""CPU checks of the decode-step counterpart (C5): layer order with a stand-in
cache, RoPE and rmsnorm closed forms, and the sampling rules of the
reference runtime (Z/model_hub/LLM.py:63-139)."""
import math

import numpy as np
import pytest
import torch

from zoomkv_revision_amd import decode_step as ds

TINY = ds.Qwen3Geometry(layers=2, hidden=64, heads=4, kv_heads=2, head_dim=128, ffn=96, vocab=50)


class DenseCache:
    """Stand-in with polar_cache's decode interface: full fp32 attention over
    every appended row (the reference's Full_Flash_Attn decode)."""

    def __init__(self, layers, bs, kv):
        self.context = 0
        self.k = [torch.zeros(bs, 0, kv, 128) for _ in range(layers)]
        self.v = [torch.zeros(bs, 0, kv, 128) for _ in range(layers)]
        self.layers = layers

    def decode_update_kv_cache(self, k, v, ldx):
        self.k[ldx] = torch.cat([self.k[ldx], k.float()], 1)
        self.v[ldx] = torch.cat([self.v[ldx], v.float()], 1)
        if ldx == self.layers - 1:
            self.context += 1
        return None, None

    def compute(self, q, ldx):
        bs, _, hq, d = q.shape
        kv = self.k[ldx].shape[2]
        k = self.k[ldx].repeat_interleave(hq // kv, dim=2)
        v = self.v[ldx].repeat_interleave(hq // kv, dim=2)
        s = torch.einsum("bqhd,bnhd->bhn", q.float(), k) / math.sqrt(d)
        o = torch.einsum("bhn,bnhd->bhd", s.softmax(-1), v)
        return o.unsqueeze(1).to(q.dtype)


def test_rms_norm_closed_form():
    x = torch.randn(3, 64).to(torch.bfloat16)
    w = torch.rand(64).to(torch.bfloat16) + 0.5
    got = ds.rms_norm(x, w, 1e-6).float()
    xf = x.double()
    ref = xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert torch.allclose(got.double(), ref, rtol=2 ** -7, atol=1e-6)


def test_rope_is_a_rotation_and_matches_rotate_half():
    m = ds.RandomQwen3(TINY, "cpu", seed=1, max_position=64)
    x = torch.randn(2, 1, 4, 128)
    for pos in (0, 5, 63):
        y = m._rope(x, pos)
        # norm-preserving per head; position 0 is the identity
        assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), rtol=1e-5)
        inv = 1.0 / (TINY.rope_theta ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
        ang = pos * inv
        x1, x2 = x[..., :64].double(), x[..., 64:].double()
        ref = torch.cat([x1 * ang.cos() - x2 * ang.sin(), x2 * ang.cos() + x1 * ang.sin()], -1)
        assert torch.allclose(y.double(), ref, atol=1e-4)
    assert torch.equal(m._rope(x, 0), x)


def test_decode_step_runs_layers_in_order_and_advances_context():
    torch.manual_seed(0)
    m = ds.RandomQwen3(TINY, "cpu", seed=3, max_position=64)
    cache = DenseCache(TINY.layers, 2, TINY.kv_heads)
    tok = torch.tensor([1, 7])
    for step in range(3):
        logits = m.decode_step(tok, cache)
        assert logits.shape == (2, TINY.vocab) and torch.isfinite(logits).all()
        assert cache.context == step + 1
        assert all(k.shape[1] == step + 1 for k in cache.k)
        tok = ds.sample_next_token(logits, 0.0)
    # the first appended key of layer 0 is rope(k_norm(W_k x)) at position 0 = k_norm(W_k x)
    L = m.layers[0]
    x = ds.rms_norm(m.embed[torch.tensor([1, 7])].unsqueeze(1), L["input_ln"], TINY.eps)
    qkv = torch.nn.functional.linear(x, L["wqkv"])
    k0 = qkv[..., 4 * 128:6 * 128].reshape(2, 1, 2, 128)
    k0 = ds.rms_norm(k0, L["k_norm"], TINY.eps)
    assert torch.equal(cache.k[0][:, :1], k0.float())


def test_sampling_rules():
    g = torch.Generator().manual_seed(42)
    logits = torch.tensor([[3.0, 1.0, 0.5, -1.0, 2.0]])
    assert ds.sample_next_token(logits, 0.0).item() == 0                 # greedy
    assert ds.sample_next_token(logits, 1.0, top_k=1, generator=g).item() == 0
    assert ds.sample_next_token(logits, 1.0, top_p=1e-6, generator=g).item() == 0
    draws = {ds.sample_next_token(logits, 1.0, top_k=2, generator=g).item() for _ in range(200)}
    assert draws == {0, 4}                                               # only the top 2
    # top-p keeps the token that crosses p: softmax(3, 2, ...) -> p0 ~ 0.64, p0 + p4 ~ 0.88
    draws = {ds.sample_next_token(logits, 1.0, top_p=0.7, generator=g).item() for _ in range(200)}
    assert draws == {0, 4}
    # seeded draws repeat
    a = [ds.sample_next_token(logits, 0.6, 0.95, 20, torch.Generator().manual_seed(42)).item() for _ in range(3)]
    assert len(set(a)) == 1


@pytest.mark.parametrize("temperature,top_p,top_k", [(0.6, 0.95, 20), (1.0, 0.5, 5), (0.8, 0.0, 50),
                                                     (1.3, 0.99, 1), (0.6, 0.95, 0)])
def test_windowed_sampling_matches_full_vocabulary(temperature, top_p, top_k):
    """The windowed sampler draws the same token as the op-for-op restatement
    of LLM.py:63-139 from the same generator state, over rows where the kept
    set is a handful of tokens (peaked logits) and where it is all of top-k."""
    gen = torch.Generator().manual_seed(7)
    for trial in range(60):
        scale = (0.5, 3.0, 12.0)[trial % 3]
        logits = torch.randn(4, 3000, generator=gen) * scale
        s = 1000 + trial
        a = ds.sample_next_token(logits, temperature, top_p, top_k, torch.Generator().manual_seed(s))
        b = ds.sample_next_token_full(logits, temperature, top_p, top_k, torch.Generator().manual_seed(s))
        assert torch.equal(a, b), (trial, a, b)


def test_windowed_sampling_ties_at_kth_value():
    """Ties at the k-th value are all kept by top-k: inside the window they are
    drawn like any kept token; a tie group larger than the window takes the
    full-vocabulary path (same draws either way)."""
    for n_ties in (3, 40):
        logits = torch.full((2, 500), -5.0)
        logits[:, :4] = torch.tensor([4.0, 3.0, 2.5, 2.0])
        logits[:, 100:100 + n_ties] = 1.0           # k = 6: tokens 4.. tie at the 6th value
        seen = set()
        for s in range(300):
            a = ds.sample_next_token(logits, 1.0, 0.999, 6, torch.Generator().manual_seed(s))
            b = ds.sample_next_token_full(logits, 1.0, 0.999, 6, torch.Generator().manual_seed(s))
            assert torch.equal(a, b)
            seen.update(a.tolist())
        assert seen <= {0, 1, 2, 3} | set(range(100, 100 + n_ties)) and len(seen & set(range(100, 200))) > 1


def test_production_env_matches_reference_runner(monkeypatch):
    # setenv records each variable's prior state (set or absent), so teardown
    # restores it whatever apply_production_env sets or pops
    for k in list(ds.PRODUCTION_ENV) + ["POLAR_FORCE_CAND_TOKENS"]:
        monkeypatch.setenv(k, "unset-by-test")
    ds.apply_production_env()
    assert "POLAR_FORCE_CAND_TOKENS" not in __import__("os").environ
    import os
    assert os.environ["POLAR_QUEST_CHUNK"] == "16"
    assert os.environ["POLAR_QUEST_DYNAMIC_CAND_RATIOS"] == "0.7,0.5,0.4"
    assert os.environ["POLAR_CDS_DENSE_RATIO"] == "0.3"
    assert ds.PRODUCTION_CACHE_KNOBS["final_topk"] == 100
