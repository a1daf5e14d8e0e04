"""The polar_cache drop-in against the CPU cache model: the same prefill and
decode steps (crossing several flushes with a chunk carry and a live skipped
tail) must give the same bookkeeping, the same selected token indices (exact)
and attention outputs within 2e-3, layer by layer and step by step."""
import numpy as np
import pytest
import torch

from oracle.cache_model import CacheModel
from tests.helpers import from_torch, gaussian_bf16, to_bf16

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _make(monkeypatch, chunk, cand, dense_ratio, dense_topk, sparse_topk, **geo):
    from zoomkv_revision_amd.cache import polar_cache
    monkeypatch.setenv("POLAR_QUEST_CHUNK", str(chunk))
    monkeypatch.setenv("POLAR_QUEST_CAND_RATIO", str(cand))
    monkeypatch.setenv("POLAR_CDS_DENSE_RATIO", str(dense_ratio))
    monkeypatch.setenv("POLAR_CDS_DENSE_TOPK", str(dense_topk))
    monkeypatch.setenv("POLAR_CDS_SPARSE_TOPK", str(sparse_topk))
    # the cache model uses the fixed candidate ratio: pin the environment to it
    monkeypatch.setenv("POLAR_QUEST_DYNAMIC_CAND_RATIO", "0")
    monkeypatch.delenv("POLAR_FORCE_CAND_TOKENS", raising=False)
    g = dict(geo)
    cache = polar_cache(
        valid_start=[0] * g["bs"], layer_num=g["L"], batch_size=g["bs"], max_length=g["inp"] + g["new"],
        num_key_value_heads=g["kv"], num_heads=g["hq"], head_dim=128, dtype=torch.bfloat16,
        layer_mapping={"0": "cuda:0"}, max_new_length=g["new"], sink_size=g["sink"], local_size=g["local"],
        core=1, nprobe=1, cache_unit_size=1, cache_cluster_num=1, num_gpus=1, model_size=8,
        final_topk=g["topk"], dynamic_update_interval=g["interval"], full_attention_threshold=g["thr"])
    model = CacheModel(g["L"], g["bs"], g["kv"], g["hq"], g["inp"], g["new"], g["sink"], g["local"], g["interval"],
                       chunk, g["topk"], g["thr"], cand, dense_ratio, dense_topk, sparse_topk)
    return cache, model


def _run(rng, cache, model, g, prompt, steps, lockstep=True):
    L, bs, kv, hq = g["L"], g["bs"], g["kv"], g["hq"]
    for l in range(L):
        k = gaussian_bf16(rng, (bs, prompt, kv, 128), outlier_channels=2)
        v = gaussian_bf16(rng, (bs, prompt, kv, 128))
        q = gaussian_bf16(rng, (bs, prompt, hq, 128))
        if lockstep:
            ko, vo = cache.prefill_update_kv_cache(to_bf16(q), to_bf16(k), to_bf16(v), l, 0)
        else:
            for b in range(bs):
                ko, vo = cache.prefill_update_kv_cache(to_bf16(q[b:b + 1]), to_bf16(k[b:b + 1]),
                                                       to_bf16(v[b:b + 1]), l, b)
        cache.sync(l, 0)
        assert ko.shape[1] == prompt
        model.prefill(k, v, l)
    assert cache.context == model.context == prompt
    n_selected = 0
    for step in range(steps):
        for l in range(L):
            k = gaussian_bf16(rng, (bs, 1, kv, 128), outlier_channels=2)
            v = gaussian_bf16(rng, (bs, 1, kv, 128))
            q = gaussian_bf16(rng, (bs, 1, hq, 128))
            assert cache.decode_update_kv_cache(to_bf16(k), to_bf16(v), l) == (None, None)
            model.decode_update(k, v, l)
            out = from_torch(cache.compute(to_bf16(q), l))
            ref, sel = model.compute(q, l)
            assert out.shape == (bs, 1, hq, 128)
            got_sel = cache._last_topk_indices
            if sel is None:
                assert got_sel is None, f"step {step} layer {l}: expected full attention"
            else:
                n_selected += 1
                assert np.array_equal(from_torch(got_sel), sel), f"step {step} layer {l}: selection"
            err = np.abs(out[:, 0] - ref).max()
            assert err <= ATOL + np.abs(ref).max() * 2 ** -8, f"step {step} layer {l}: err {err}"
        assert cache.cpu_valid_end == model.cpu_valid_end, f"step {step}"
        assert cache._chunk_carry_count == model.carry and cache.context == model.context
        assert cache._chunk_skipped_count[0] == len(model.skipped)
    return n_selected


GEO = dict(L=2, bs=2, kv=2, hq=8, inp=400, new=200, sink=4, local=64, interval=32, topk=16, thr=0)


def test_cache_trace_chunk8_with_carry_and_flushes(rng, monkeypatch):
    # retrieval after prefill: 400 - 4 - 64 = 332 = 41 chunks + 4 carried tokens
    cache, model = _make(monkeypatch, 8, 0.2, 0.3, 8, 4, **GEO)
    n = _run(rng, cache, model, GEO, prompt=400, steps=110)
    assert n == 2 * 110 and cache.cpu_valid_end[0] == 332 + 3 * 32


def test_cache_trace_chunk16_single_sample_prefill(rng, monkeypatch):
    geo = dict(GEO, inp=300, thr=380)       # full attention first, then retrieval after a flush
    cache, model = _make(monkeypatch, 16, 0.3, 0.3, 16, 8, **geo)
    n = _run(rng, cache, model, geo, prompt=300, steps=90, lockstep=False)
    assert 0 < n < 2 * 90


def test_cache_trace_equal_dense_sparse_topk(rng, monkeypatch):
    # the production knobs (dense = sparse = 8): the density classification is
    # skipped, the selection must still equal the model's, which computes it
    cache, model = _make(monkeypatch, 16, 0.4, 0.3, 8, 8, **GEO)
    n = _run(rng, cache, model, GEO, prompt=400, steps=70)
    assert n == 2 * 70


def test_cache_short_prompt_full_attention(rng, monkeypatch):
    geo = dict(GEO, inp=50, new=60)
    cache, model = _make(monkeypatch, 8, 0.2, 0.3, 8, 8, **geo)
    assert _run(rng, cache, model, geo, prompt=50, steps=40) == 0


def test_cache_module_is_selectable_by_name():
    """The runtime resolves importlib.import_module(name).polar_cache and
    filters its kwargs by the constructor signature (Z/model_hub/qwen.py:336-419)."""
    import importlib
    import inspect
    cls = importlib.import_module("zoomkv_revision_amd.cache").polar_cache
    params = inspect.signature(cls.__init__).parameters
    for key in ("valid_start", "layer_num", "batch_size", "max_length", "num_key_value_heads", "num_heads",
                "head_dim", "dtype", "layer_mapping", "max_new_length", "sink_size", "local_size", "core",
                "nprobe", "cache_unit_size", "cache_cluster_num", "num_gpus", "model_size", "collision_ratio",
                "candidate_ratio", "enable_offload", "dynamic_update_interval", "codebook_path", "final_topk",
                "full_attention_threshold"):
        assert key in params, key
