"""Configuration C5 at its own geometry: one decode token of a 36-layer
Qwen3-4B-geometry model (hidden 2560, 32 / 8 heads of 128, FFN 9728,
vocabulary 151936, random-init bf16 weights) through polar_cache at a
65536-token context, batch 4, with the reference runner's production knobs
(chunk 16, dynamic candidate ratio -> 1631 candidate chunks of 4076, CDS
dense = sparse top-k 8, top-100, sink 64, local 256, interval 512).

For the first and the last layer:
* Format R metadata (chunk min / max / centroid, 4-bit codes, valid) of the
  first and last 64 chunks equals the oracle's encode of the stored keys;
* the selected token indices equal the oracle's selection recomputed from the
  recorded query and the cache's metadata (GQA mean -> Quest -> top-nk ->
  density -> dense mask -> KIVI stage 2 -> top-100 + skipped), exactly;
* the attention output is within 2e-3 (+ the bf16 output rounding) of float64
  attention over sink + local + the selected rows;
and the whole fused layer (QKV with the RMSNorm, q / k norm + RoPE, the
attention, o-projection, MLP) matches the torch ops of the reference's
layer_decode on the same input and attention output.

The last test then decodes on to the first flush (512 tokens past the
prompt's local window): the flushed rows are the local tokens they were, the
32 newly encoded chunks' metadata equals the oracle's encode of them, and the
flush step's selection and attention match the oracle as above."""
import numpy as np
import pytest
import torch

from oracle import kivi as okivi
from oracle import select as osel
from oracle.kivi import encode_chunks_ref
from tests.helpers import from_torch

pytestmark = pytest.mark.gpu

LAYERS = (0, 35)
BATCH, CONTEXT, INTERVAL, THRESHOLD = 4, 65536, 512, 2048
MAX_NEW = INTERVAL + 8          # room for the decode steps up to the first flush


@pytest.fixture(scope="module")
def c5(request):
    from zoomkv_revision_amd import decode_step as ds
    mp = pytest.MonkeyPatch()
    for k, v in ds.PRODUCTION_ENV.items():
        mp.setenv(k, v)
    mp.delenv("POLAR_FORCE_CAND_TOKENS", raising=False)
    geo = ds.Qwen3Geometry()
    dev = torch.device("cuda:0")
    model = ds.RandomQwen3(geo, dev, seed=42)
    cache = ds.build_cache(geo, BATCH, CONTEXT, MAX_NEW, INTERVAL, THRESHOLD, dev)
    ds.fill_cache(cache, geo, BATCH, CONTEXT, 43, dev)
    rec = {l: {} for l in LAYERS}
    compute, layer = cache.compute, model.layer_decode

    def compute_rec(queries, layer_idx):
        out = compute(queries, layer_idx)
        if layer_idx in rec:
            rec[layer_idx].update(q=queries.clone(), out=out.clone(), idx=cache._last_topk_indices.clone(),
                                  near_len=cache.sink_size + cache.get_region_indices(layer_idx)["local_len"])
        return out

    def layer_rec(ldx, hidden, c):
        h_out = layer(ldx, hidden, c)
        if ldx in rec:
            rec[ldx].update(h_in=hidden.clone(), h_out=h_out.clone())
        return h_out

    cache.compute, model.layer_decode = compute_rec, layer_rec
    tok = torch.tensor([11, 2024, 77, 150000], device=dev)
    logits = model.decode_step(tok, cache)
    torch.cuda.synchronize()
    yield {"ds": ds, "geo": geo, "model": model, "cache": cache, "rec": rec, "logits": logits}
    mp.undo()
    del cache, model
    torch.cuda.empty_cache()


def _np(t):
    return from_torch(t.float()) if t.dtype == torch.bfloat16 else from_torch(t)


@pytest.mark.parametrize("layer", LAYERS)
def test_c5_metadata_and_selection_match_oracle(c5, layer):
    cache, rec = c5["cache"], c5["rec"][layer]
    assert torch.isfinite(c5["logits"]).all()
    L = int(cache.cpu_valid_end[layer])
    chunk = cache.quest_chunk_size
    n_chunks, nk = cache._cached_quest_n_chunks, cache._cached_quest_nk
    assert (L, chunk, n_chunks, nk) == (CONTEXT - 64 - 256, 16, (CONTEXT - 320) // 16, 1631)
    _check_selection_and_attention(cache, rec, layer, (0, n_chunks - 64))


def _check_selection_and_attention(cache, rec, layer, chunk_starts):
    """Format R metadata of 64 chunks from each of ``chunk_starts`` against the
    oracle's encode of the stored keys, the recorded selection against the
    oracle's, and the recorded attention output against float64 attention
    over sink + local + the selected rows."""
    L = int(cache.cpu_valid_end[layer])
    chunk = cache.quest_chunk_size
    n_chunks, nk = cache._cached_quest_n_chunks, cache._cached_quest_nk
    mn = _np(cache._chunk_key_min_gpu[layer])
    mx = _np(cache._chunk_key_max_gpu[layer])
    mean = _np(cache._chunk_key_centroid_gpu[layer])
    valid = _np(cache._chunk_valid_mask_gpu[layer]).astype(bool)
    packed = _np(cache.key_kivi_packed_gpu[layer])
    assert valid[:, :, :n_chunks].all() and not valid[:, :, n_chunks:].any()
    for c0 in chunk_starts:
        keys = _np(cache.unified_keys[layer][:, :, c0 * chunk:(c0 + 64) * chunk])
        rmn, rmx, rmean, rpk = encode_chunks_ref(keys, chunk)
        sl = slice(c0, c0 + 64)
        assert np.array_equal(mn[:, :, sl], rmn) and np.array_equal(mx[:, :, sl], rmx)
        assert np.array_equal(mean[:, :, sl], rmean) and np.array_equal(packed[:, :, sl], rpk)
    # the oracle's selection from the recorded query (S:2195-2467, S:2688-2779)
    raw_q = osel.gqa_mean_query(_np(rec["q"])[:, 0], cache.kv_head)
    sc = osel.quest_chunk_score(raw_q, mn, mx, n_chunks, valid)
    cidx = np.clip(osel.topk_indices(sc, nk), 0, n_chunks - 1)
    dens = osel.chunk_density_scores(cidx, mean, raw_q)
    dmask = osel.dense_mask_from_topk(osel.topk_indices(dens, cache._cached_cds_n_dense), nk)
    s2, i2 = osel.kivi_qk_dense_sparse(cidx, dmask, packed[:, :, :L // chunk], mn, mx, raw_q, 8, 8, chunk)
    sk = cache._chunk_skipped_count[layer]
    skipped = np.broadcast_to(np.arange(n_chunks * chunk, L), (BATCH, cache.kv_head, sk))
    want = osel.topk_gather_concat(s2, i2, skipped, 100, 100 + sk)
    got = _np(rec["idx"])
    assert got.shape == want.shape and np.array_equal(got, want)
    # attention over sink + local + the selected rows (float64)
    K, V = cache.unified_keys[layer], cache.unified_values[layer]
    near = slice(cache._near0, cache._near0 + rec["near_len"])
    q = _np(rec["q"])[:, 0]
    out = _np(rec["out"])[:, 0]
    g = cache.num_heads // cache.kv_head
    for b in range(BATCH):
        for h in range(cache.kv_head):
            rows = torch.from_numpy(want[b, h]).to(K.device)
            kk = torch.cat([K[b, h, rows], K[b, h, near]]).float().cpu().numpy()
            vv = torch.cat([V[b, h, rows], V[b, h, near]]).float().cpu().numpy()
            ref = okivi.attention(q[b:b + 1, h * g:(h + 1) * g], kk[None, None], vv[None, None], 1 / np.sqrt(128))[0]
            o = out[b, h * g:(h + 1) * g]
            assert np.abs(o - ref).max() <= 2e-3 + np.abs(ref).max() * 2 ** -8, (b, h)


@pytest.mark.parametrize("layer", LAYERS)
def test_c5_fused_layer_matches_torch_ops(c5, layer):
    """The five fused launches of the layer against layer_decode's torch ops
    (Z/model_hub/LLM.py:208-251) on the same input hidden state and the same
    attention output, within a few bf16 units at each tensor's scale."""
    import torch.nn.functional as F
    ds, geo, model, rec = c5["ds"], c5["geo"], c5["model"], c5["rec"][layer]
    W = model.layers[layer]
    h_in = rec["h_in"]
    bs = h_in.shape[0]
    qd, kd = geo.heads * geo.head_dim, geo.kv_heads * geo.head_dim
    x = ds.rms_norm(h_in, W["input_ln"], geo.eps)
    qkv = F.linear(x, W["wqkv"])
    q, k, v = qkv.split([qd, kd, kd], dim=-1)
    pos = CONTEXT                                           # the token's position
    q = model._rope(ds.rms_norm(q.reshape(bs, 1, geo.heads, geo.head_dim), W["q_norm"], geo.eps), pos)

    def close(got, ref, ulps):
        got, ref = got.float(), ref.float()
        tol = ulps * ref.abs().max().item() * 2.0 ** -7 + 1e-6
        assert (got - ref).abs().max().item() <= tol

    close(rec["q"], q, 4.0)
    attn = rec["out"]
    hidden = h_in + F.linear(attn.reshape(bs, 1, qd), W["wo"])
    x2 = ds.rms_norm(hidden, W["post_ln"], geo.eps)
    gate, up = F.linear(x2, W["gate_up"]).chunk(2, dim=-1)
    h_ref = hidden + F.linear(F.silu(gate) * up, W["down"])
    close(rec["h_out"], h_ref, 8.0)


def test_c5_first_flush_matches_oracle(c5):
    """Runs last (it moves the cache on): decode until the step whose layer 0
    flushes the oldest 512 local tokens into the retrieval zone.  Then, for
    the first and last layer, the 512 new retrieval rows are bit-identical to
    the local rows they came from, the 32 new chunks' Format R metadata
    equals the oracle's encode of them, the stage-1 sizes follow the new
    retrieval length, and the flush step's selection and attention match the
    oracle (as at the prompt's end)."""
    cache, model, rec = c5["cache"], c5["model"], c5["rec"]
    L0 = int(cache.cpu_valid_end[0])
    s, n0 = cache.sink_size, cache._near0
    oldest = slice(n0 + s, n0 + s + INTERVAL)
    tok = c5["logits"].argmax(dim=-1)
    moved, steps = None, 0
    while int(cache.cpu_valid_end[0]) == L0:
        near_len = cache.current_seq_len[0] - s - L0
        if near_len >= cache.local_size + INTERVAL:          # this step's layer 0 flushes
            moved = {l: (cache.unified_keys[l][:, :, oldest].clone(), cache.unified_values[l][:, :, oldest].clone())
                     for l in LAYERS}
        tok = model.decode_step(tok, cache).argmax(dim=-1)
        steps += 1
        assert steps <= INTERVAL + 1, "no flush"
    torch.cuda.synchronize()
    print(f"[c5 flush] flushed after {steps} more decode steps", flush=True)
    L1 = L0 + INTERVAL
    assert moved is not None and all(int(e) == L1 for e in cache.cpu_valid_end)
    chunk = cache.quest_chunk_size
    assert cache._cached_quest_n_chunks == L1 // chunk
    # nk of S:1798-1825 at the new length (dynamic ratio 0.4 above 10001 tokens)
    assert cache._cached_quest_nk == min(L1 // chunk, -(-int(np.ceil(L1 * 0.4)) // chunk))
    for layer in LAYERS:
        k_old, v_old = moved[layer]
        assert torch.equal(cache.unified_keys[layer][:, :, L0:L1], k_old)
        assert torch.equal(cache.unified_values[layer][:, :, L0:L1], v_old)
        rmn, rmx, rmean, rpk = encode_chunks_ref(_np(k_old), chunk)
        new = slice(L0 // chunk, L1 // chunk)
        assert np.array_equal(_np(cache._chunk_key_min_gpu[layer])[:, :, new], rmn)
        assert np.array_equal(_np(cache._chunk_key_max_gpu[layer])[:, :, new], rmx)
        assert np.array_equal(_np(cache._chunk_key_centroid_gpu[layer])[:, :, new], rmean)
        assert np.array_equal(_np(cache.key_kivi_packed_gpu[layer])[:, :, new], rpk)
        _check_selection_and_attention(cache, rec[layer], layer, (0, L0 // chunk - 32))
