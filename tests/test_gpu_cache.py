"""The polar_cache drop-in against the CPU cache model: the same prefill and
decode steps (crossing several flushes with a chunk carry and a live skipped
tail) must give the same bookkeeping, the same selected token indices (exact)
and attention outputs within 2e-3, layer by layer and step by step -- with the
retrieval zone in pinned host memory (enable_offload=True) and in device
memory (False), and as the 4-bit K + V retrieval zone (kv_format "kivi4",
Format Q groups plus a bf16 tail, attended by the token-list kernel) against
the model's dequantized rows; the two bf16 modes give identical selections
and outputs."""
import numpy as np
import pytest
import torch

from oracle.cache_model import CacheModel
from tests.helpers import from_torch, gaussian_bf16, to_bf16

pytestmark = pytest.mark.gpu

ATOL = 2e-3


STORAGE = ["offload", "device", "kivi4"]


def _make(monkeypatch, chunk, cand, dense_ratio, dense_topk, sparse_topk, offload=True, storage=None, **geo):
    kv_format = "bf16"
    if storage is not None:
        offload, kv_format = storage == "offload", ("kivi4" if storage == "kivi4" else "bf16")
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
        final_topk=g["topk"], dynamic_update_interval=g["interval"], full_attention_threshold=g["thr"],
        enable_offload=offload, kv_format=kv_format)
    assert (cache.unified_keys_cpu is not None) == (offload and kv_format == "bf16")
    if kv_format == "kivi4":   # device rows = 32 tail rows + near zone
        assert cache.unified_keys[0].shape[2] == 32 + cache.gpu_kv_capacity
    elif offload:   # host retrieval zone; device rows = gather area + near zone
        assert cache.unified_keys_cpu[0].is_pinned()
        assert cache.unified_keys[0].shape[2] == cache._gather_rows + cache.gpu_kv_capacity
    model = CacheModel(g["L"], g["bs"], g["kv"], g["hq"], g["inp"], g["new"], g["sink"], g["local"], g["interval"],
                       chunk, g["topk"], g["thr"], cand, dense_ratio, dense_topk, sparse_topk, kv_format=kv_format)
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


@pytest.mark.parametrize("storage", STORAGE)
def test_cache_trace_chunk8_with_carry_and_flushes(rng, monkeypatch, storage):
    # retrieval after prefill: 400 - 4 - 64 = 332 = 41 chunks + 4 carried tokens
    # (kivi4: 10 groups + a 12-token bf16 tail, through every flush)
    cache, model = _make(monkeypatch, 8, 0.2, 0.3, 8, 4, storage=storage, **GEO)
    n = _run(rng, cache, model, GEO, prompt=400, steps=110)
    assert n == 2 * 110 and cache.cpu_valid_end[0] == 332 + 3 * 32


@pytest.mark.parametrize("storage", STORAGE)
def test_cache_trace_chunk16_single_sample_prefill(rng, monkeypatch, storage):
    geo = dict(GEO, inp=300, thr=380)       # full attention first, then retrieval after a flush
    cache, model = _make(monkeypatch, 16, 0.3, 0.3, 16, 8, storage=storage, **geo)
    n = _run(rng, cache, model, geo, prompt=300, steps=90, lockstep=False)
    assert 0 < n < 2 * 90


@pytest.mark.parametrize("storage", STORAGE)
def test_cache_trace_equal_dense_sparse_topk(rng, monkeypatch, storage):
    # the production knobs (dense = sparse = 8): the density classification is
    # skipped, the selection must still equal the model's, which computes it
    cache, model = _make(monkeypatch, 16, 0.4, 0.3, 8, 8, storage=storage, **GEO)
    n = _run(rng, cache, model, GEO, prompt=400, steps=70)
    assert n == 2 * 70


@pytest.mark.parametrize("storage", STORAGE)
def test_cache_short_prompt_full_attention(rng, monkeypatch, storage):
    geo = dict(GEO, inp=50, new=60)
    cache, model = _make(monkeypatch, 8, 0.2, 0.3, 8, 8, storage=storage, **geo)
    assert _run(rng, cache, model, geo, prompt=50, steps=40) == 0


def test_cache_kivi4_aligned_retrieval_and_threshold(rng, monkeypatch):
    """kivi4 storage with a 32-aligned retrieval zone (no bf16 tail: flushes
    pack straight from the near zone) and the full-attention threshold
    crossed during decode (dense 4-bit kernel, then the token-list kernel)."""
    geo = dict(GEO, inp=388, new=160, thr=470)   # retrieval 388 - 68 = 320 = 10 groups
    cache, model = _make(monkeypatch, 16, 0.3, 0.3, 16, 8, storage="kivi4", **geo)
    n = _run(rng, cache, model, geo, prompt=388, steps=120)
    assert 0 < n < 2 * 120 and cache.cpu_valid_end[0] % 32 == 0
    cache.check_range()


def test_cache_kivi4_stores_no_bf16_retrieval_rows(monkeypatch):
    """kivi4 storage keeps the retrieval zone as Format Q records only: the
    device rows are the 32-row tail plus the near zone (no gather area, no
    host rows), and the records take 160 B per token per KV head."""
    geo = dict(GEO, inp=400, new=200)
    cache, _ = _make(monkeypatch, 16, 0.3, 0.3, 16, 8, storage="kivi4", **geo)
    cap = cache.cpu_kv_capacity
    assert cache.unified_keys_cpu is None and cache.unified_keys[0].shape[2] == 32 + cache.gpu_kv_capacity
    g = cache.kivi4_groups[0]
    assert g.shape[2] == (cap + 31) // 32 and g.element_size() * g.shape[3] == 32 * 160


def test_cache_offload_modes_identical(rng, monkeypatch):
    """Host-resident and device-resident retrieval zones, fed the same prompt
    and tokens through three flushes: identical selections, identical
    attention outputs (bit for bit) and the same retrieval-zone contents."""
    geo = dict(GEO, inp=300, new=160, thr=330)
    host, _ = _make(monkeypatch, 16, 0.3, 0.3, 16, 8, offload=True, **geo)
    dev, _ = _make(monkeypatch, 16, 0.3, 0.3, 16, 8, offload=False, **geo)
    L, bs, kv, hq = geo["L"], geo["bs"], geo["kv"], geo["hq"]
    for l in range(L):
        k, v = (to_bf16(gaussian_bf16(rng, (bs, 300, kv, 128))) for _ in range(2))
        for c in (host, dev):
            c.prefill_update_kv_cache(None, k, v, l, 0)
    selected = 0
    for step in range(120):
        for l in range(L):
            k, v, q = (to_bf16(gaussian_bf16(rng, (bs, 1, n, 128))) for n in (kv, kv, hq))
            outs = []
            for c in (host, dev):
                c.decode_update_kv_cache(k, v, l)
                outs.append(c.compute(q, l))
            assert torch.equal(outs[0], outs[1]), f"step {step} layer {l}"
            a, b = host._last_topk_indices, dev._last_topk_indices
            assert (a is None) == (b is None) and (a is None or torch.equal(a, b)), f"step {step} layer {l}"
            selected += a is not None
    torch.cuda.synchronize()
    assert host.cpu_valid_end == dev.cpu_valid_end and host.cpu_valid_end[0] == 300 - 4 - 64 + 3 * 32
    assert selected > 0
    for l in range(L):
        n = host.cpu_valid_end[l]
        assert torch.equal(host.unified_keys_cpu[l][:, :, :n], dev.unified_keys[l][:, :, :n].cpu())
        assert torch.equal(host.unified_values_cpu[l][:, :, :n], dev.unified_values[l][:, :, :n].cpu())


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
