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
    assert b["total"] > b["quest_gqa"] > 0


def test_windowed_sampling_matches_full_vocabulary_on_device():
    """On the device generator: the windowed sampler and the op-for-op
    restatement of LLM.py:63-139 draw the same tokens over a Qwen3-size
    vocabulary (both consume one Exp(1) row per draw, so the streams stay
    aligned across calls)."""
    g = torch.Generator(device="cuda").manual_seed(3)
    ga = torch.Generator(device="cuda").manual_seed(11)
    gb = torch.Generator(device="cuda").manual_seed(11)
    for trial in range(40):
        logits = torch.randn(4, 151936, generator=g, device="cuda") * (0.5, 4.0, 16.0, 40.0)[trial % 4]
        a = ds.sample_next_token(logits, 0.6, 0.95, 20, generator=ga)
        b = ds.sample_next_token_full(logits, 0.6, 0.95, 20, generator=gb)
        assert torch.equal(a, b), (trial, a, b)


@pytest.mark.parametrize("bs,vocab", [(4, 151936), (1, 8192 + 10), (3, 100), (8, 3000), (2, 16384)])
@pytest.mark.parametrize("temperature,top_p,top_k", [(0.6, 0.95, 20), (1.0, 0.5, 5), (0.8, 0.0, 48),
                                                     (1.3, 0.99, 1)])
def test_hip_sampler_matches_full_vocabulary(bs, vocab, temperature, top_p, top_k):
    """The one-launch sampler (zkv_sample_window) against the op-for-op
    restatement of LLM.py:63-139 from the same device generator state: vocab
    sizes with a slice shorter than the window (8202), single slices (100,
    3000) and exact multiples; peaked and flat rows."""
    if top_k + 16 >= vocab:
        pytest.skip("the window covers the vocabulary: the full path runs")
    g = torch.Generator(device="cuda").manual_seed(vocab + top_k)
    ga = torch.Generator(device="cuda").manual_seed(5)
    gb = torch.Generator(device="cuda").manual_seed(5)
    for trial in range(12):
        logits = torch.randn(bs, vocab, generator=g, device="cuda") * (0.5, 4.0, 16.0)[trial % 3]
        a = ds.sample_next_token(logits, temperature, top_p, top_k, generator=ga)
        b = ds.sample_next_token_full(logits, temperature, top_p, top_k, generator=gb)
        assert a.dtype == torch.int64 and a.shape == (bs,)
        assert torch.equal(a, b), (trial, a, b)
        # the launch itself (no tie overflow on these rows, so no full-vocabulary draw)
        expo = torch.empty_like(logits).exponential_(1, generator=g)
        tok, flags = ds.sample_window_launch(logits, temperature, top_p, top_k, expo)
        assert int(flags.abs().sum()) == 0
        assert torch.equal(tok, ds.draw_full_vocabulary(logits, temperature, top_p, top_k, expo)), trial


def test_hip_sampler_ties_at_kth_value():
    """Ties at the k-th value: a group inside the window is drawn like any
    kept token; one wider than the window sets the row's overflow flag and the
    draw runs over the whole vocabulary with the same Exp(1) row."""
    for n_ties in (3, 40):
        logits = torch.full((2, 20000), -5.0, device="cuda")
        logits[:, 7:11] = torch.tensor([4.0, 3.0, 2.5, 2.0], device="cuda")
        logits[:, 9000:9000 + n_ties] = 1.0           # k = 6: the 6th value is a tie
        expo = torch.empty_like(logits).exponential_(1)
        _, flags = ds.sample_window_launch(logits, 1.0, 0.999, 6, expo)
        assert flags.tolist() == [int(n_ties > 16)] * 2
        ga = torch.Generator(device="cuda").manual_seed(1)
        gb = torch.Generator(device="cuda").manual_seed(1)
        seen = set()
        for _ in range(200):
            a = ds.sample_next_token(logits, 1.0, 0.999, 6, generator=ga)
            b = ds.sample_next_token_full(logits, 1.0, 0.999, 6, generator=gb)
            assert torch.equal(a, b)
            seen.update(a.tolist())
        assert seen <= set(range(7, 11)) | set(range(9000, 9000 + n_ties))
        assert len(seen & set(range(9000, 9000 + n_ties))) > 1


def test_hip_sampler_rejects_bad_arguments():
    from zoomkv_revision_amd._lib import ZkvError, check, lib, ptr
    L = lib()
    x = torch.randn(2, 1000, device="cuda")
    e = torch.ones_like(x)
    tok = torch.empty(2, dtype=torch.int64, device="cuda")
    fl = torch.empty(2, dtype=torch.int32, device="cuda")
    ws = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    args = lambda k, w, nbytes: (ptr(x), 1000, 2, 1000, 1.0, k, w, 0.9, ptr(e), 1000, ptr(tok), ptr(fl),
                                 ptr(ws), nbytes, 0)
    with pytest.raises(ZkvError):
        check(L.zkv_sample_window(*args(20, 65, ws.numel())))        # window over one wave
    with pytest.raises(ZkvError):
        check(L.zkv_sample_window(*args(20, 20, ws.numel())))        # window not past k
    with pytest.raises(ZkvError):
        check(L.zkv_sample_window(*args(20, 36, 16)))                # workspace too small
    check(L.zkv_sample_window(*args(20, 36, ws.numel())))
    torch.cuda.synchronize()
    assert ((tok >= 0) & (tok < 1000)).all() and (fl == 0).all()


def _bf16_close(got, ref, ulps=1.0):
    """Within `ulps` bf16 units at the tensor's largest magnitude (the fp32
    accumulation order differs from the library GEMM's)."""
    got, ref = got.float(), ref.float()
    scale = ref.abs().max().item()
    tol = ulps * scale * 2.0 ** -7 + 1e-6
    err = (got - ref).abs().max().item()
    assert err <= tol, (err, tol)


@pytest.mark.parametrize("M,K,N", [(4, 2560, 6144), (1, 512, 1000), (16, 256, 48), (4, 9728, 2560),
                                   (2, 4096, 2560), (8, 2560, 1000), (5, 256, 13), (3, 9728, 24),
                                   (8, 8192, 64), (12, 384, 40)])
def test_decode_linear_plain_and_norm(M, K, N):
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    nw = (torch.rand(K, generator=g, device="cuda") + 0.5).to(torch.bfloat16)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ds.decode_linear(x, w, out)
    _bf16_close(out, (x.float() @ w.float().T).to(torch.bfloat16))
    xn = ds.rms_norm(x, nw, 1e-6)
    ds.decode_linear(x, w, out, norm_w=nw, eps=1e-6)
    _bf16_close(out, (xn.float() @ w.float().T).to(torch.bfloat16), ulps=2.0)
    out32 = torch.empty(M, N, dtype=torch.float32, device="cuda")
    ds.decode_linear(x, w, out32, norm_w=nw, eps=1e-6)
    assert torch.equal(out32, out32.to(torch.bfloat16).float())        # bf16 values held in fp32
    assert torch.equal(out32.to(torch.bfloat16), out)


@pytest.mark.parametrize("M,K,F_", [(4, 2560, 9728), (7, 512, 37), (12, 256, 24), (6, 256, 384)])
def test_decode_linear_residual_and_silu_mul(M, K, F_):
    g = torch.Generator(device="cuda").manual_seed(5 + M)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(2 * F_, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    act = torch.empty(M, F_, dtype=torch.bfloat16, device="cuda")
    ds.decode_linear(x, w, act, silu_mul=True)
    y = (x.float() @ w.float().T).to(torch.bfloat16)
    ref = torch.nn.functional.silu(y[:, :F_]) * y[:, F_:]
    _bf16_close(act, ref, ulps=2.0)
    if F_ % 128:
        return                                           # the down projection needs K = F_ % 128 == 0
    wo = (torch.randn(K, F_, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    res = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    h = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
    ds.decode_linear(act, wo, h, residual=res)
    _bf16_close(h, res + (act.float() @ wo.float().T).to(torch.bfloat16), ulps=2.0)


def test_decode_linear_rejects_bad_shapes():
    from zoomkv_revision_amd._lib import ZkvError
    x = torch.zeros(4, 200, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(16, 200, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ZkvError):                                        # K not a multiple of 128
        ds.decode_linear(x, w, torch.empty(4, 16, dtype=torch.bfloat16, device="cuda"))


def test_qk_norm_rope_and_append_match_torch():
    geo = ds.Qwen3Geometry(layers=1, hidden=256, heads=32, kv_heads=8, head_dim=128, ffn=512, vocab=1000)
    m = ds.RandomQwen3(geo, "cuda", seed=3, max_position=4096)
    L = m.layers[0]
    L["q_norm"] = (torch.rand(128, device="cuda") + 0.5).to(torch.bfloat16)
    L["k_norm"] = (torch.rand(128, device="cuda") + 0.5).to(torch.bfloat16)
    bs, pos = 3, 3001
    qkv = torch.randn(bs, (32 + 16) * 128, device="cuda").to(torch.bfloat16)
    q = torch.empty(bs, 1, 32, 128, dtype=torch.bfloat16, device="cuda")
    K = torch.zeros(bs, 8, 40, 128, dtype=torch.bfloat16, device="cuda")
    V = torch.zeros_like(K)
    ds.qk_norm_rope(qkv, 32, 8, L["q_norm"], L["k_norm"], geo.eps, m.cos[pos], m.sin[pos], q,
                    K[:, :, 17], V[:, :, 17])
    qr, kr, vr = qkv.split([32 * 128, 8 * 128, 8 * 128], dim=-1)
    q_ref = m._rope(ds.rms_norm(qr.reshape(bs, 1, 32, 128), L["q_norm"], geo.eps), pos)
    k_ref = m._rope(ds.rms_norm(kr.reshape(bs, 1, 8, 128), L["k_norm"], geo.eps), pos)
    _bf16_close(q, q_ref, ulps=2.0)
    _bf16_close(K[:, :, 17], k_ref[:, 0], ulps=2.0)
    assert torch.equal(V[:, :, 17], vr.reshape(bs, 8, 128))
    assert not K[:, :, 16].any() and not K[:, :, 18].any()              # only the reserved row


def test_fused_decode_step_matches_torch_layers(monkeypatch):
    for k, v in ds.PRODUCTION_ENV.items():
        monkeypatch.setenv(k, v)
    monkeypatch.delenv("POLAR_FORCE_CAND_TOKENS", raising=False)
    geo = ds.Qwen3Geometry(layers=2, hidden=256, heads=32, kv_heads=8, head_dim=128, ffn=512, vocab=1000)
    dev = torch.device("cuda:0")
    batch, context = 2, 4096
    outs = []
    for fused in (True, False):
        model = ds.RandomQwen3(geo, dev, seed=42, max_position=8192, fused=fused)
        cache = ds.build_cache(geo, batch, context, 8, 64, 2048, dev)
        ds.fill_cache(cache, geo, batch, context, 43, dev)
        tok = torch.tensor([5, 77], device=dev)
        logits = [model.decode_step(tok, cache) for _ in range(3)]
        outs.append((logits, cache))
    (lf, cf), (lt, ct) = outs
    assert cf.context == ct.context == context + 3
    for a, b in zip(lf, lt):
        _bf16_close(a, b, ulps=8.0)
    row = ct._near0 + (ct.current_seq_len[0] - 1 - int(ct.cpu_valid_end[0]))
    _bf16_close(cf.unified_keys[1][:, :, row], ct.unified_keys[1][:, :, row], ulps=8.0)
