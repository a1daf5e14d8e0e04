"""Decode-step counterpart of the reference runtime for the C5 configuration.

One decode step of a Qwen3-geometry model over the drop-in ``polar_cache``,
in the order of the reference's ``layer_decode``
(Z/model_hub/LLM.py:208-251) with the layer pieces of
Z/model_hub/qwen.py:439-604:

  rmsnorm -> fused QKV linear -> per-head q / k rmsnorm -> RoPE at position
  ``cache.context`` -> ``cache.decode_update_kv_cache`` -> ``cache.compute``
  -> o-projection + residual -> rmsnorm -> gate/up linear, silu * up, down
  linear + residual;

then the final norm, the tied LM head and ``sample_next_token``
(LLM.py:63-139: temperature, top-k, top-p, multinomial).

The weights are random-init bf16 stand-ins (no checkpoint is available
offline).  On the GPU a layer is five launches besides the cache's attention
path (all in csrc/decode_model.hip): the QKV projection with the input
RMSNorm fused in, q / k norm + RoPE with the K / V rows written straight into
the cache, the o-projection with the residual add, the gate / up projection
with the post-attention RMSNorm and silu * up fused in, and the down
projection with the residual add.  The torch ops of ``layer_decode_torch``
(the reference's flashinfer rmsnorm / rope / silu have no ROCm build) are
the same layer written out op by op: the CPU path, and the check the fused
kernels are tested against.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

import torch
import torch.nn.functional as F

# The reference runner's ZoomKV environment (Z/run/eval_math_aime.py:216-238)
# and cache knobs (polar_config, :177-213), restricted to what polar_cache reads.
PRODUCTION_ENV = {
    "POLAR_QUEST_CHUNK": "16",
    "POLAR_QUEST_CAND_RATIO": "0.4",
    "POLAR_QUEST_DYNAMIC_CAND_RATIO": "1",
    "POLAR_QUEST_DYNAMIC_CAND_THRESHOLDS": "5000,10001",
    "POLAR_QUEST_DYNAMIC_CAND_RATIOS": "0.7,0.5,0.4",
    "POLAR_CDS_DENSE_RATIO": "0.3",
    "POLAR_CDS_DENSE_TOPK": "8",
    "POLAR_CDS_SPARSE_TOPK": "8",
}
PRODUCTION_CACHE_KNOBS = {"sink_size": 64, "local_size": 256, "final_topk": 100,
                          "collision_ratio": 0.3, "candidate_ratio": 0.4, "enable_offload": True}


def apply_production_env() -> None:
    """Set the reference's production ZoomKV environment (before building a cache)."""
    os.environ.update(PRODUCTION_ENV)
    os.environ.pop("POLAR_FORCE_CAND_TOKENS", None)


@dataclass(frozen=True)
class Qwen3Geometry:
    """Qwen3-4B: 36 layers, 32 / 8 heads of 128 (from the reference's
    configuration); hidden / FFN / vocabulary sizes are the public Qwen3-4B
    values, used as random-init stand-ins."""
    layers: int = 36
    hidden: int = 2560
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 9728
    vocab: int = 151936
    rope_theta: float = 1.0e6
    eps: float = 1.0e-6


def decode_linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor, norm_w: torch.Tensor | None = None,
                  eps: float = 0.0, residual: torch.Tensor | None = None, silu_mul: bool = False) -> torch.Tensor:
    """out = [silu * up of] [rmsnorm(x) of] x @ w.T [+ residual] on the GPU
    (zkv_decode_linear): x [M, K] bf16 (M <= 16), w [N, K] bf16, out [M, N]
    bf16 or fp32 (or [M, N / 2] with silu_mul: w's first half rows are gate)."""
    from ._lib import check, lib, stream_of
    M, K = x.shape
    N = w.shape[0]
    assert x.dtype == w.dtype == torch.bfloat16 and x.stride(1) == 1 and w.is_contiguous()
    assert out.dim() == 2 and out.shape[0] == M and out.shape[1] == (N // 2 if silu_mul else N)
    assert out.stride(1) == 1 and out.dtype in (torch.bfloat16, torch.float32)
    epi = 2 if silu_mul else (1 if residual is not None else 0)
    if residual is not None:
        assert residual.shape == out.shape and residual.dtype == torch.bfloat16 and residual.stride(1) == 1
    check(lib().zkv_decode_linear(x.data_ptr(), x.stride(0), M, K, w.data_ptr(), N,
                                  None if norm_w is None else norm_w.data_ptr(), float(eps),
                                  None if residual is None else residual.data_ptr(),
                                  0 if residual is None else residual.stride(0), out.data_ptr(), out.stride(0),
                                  int(out.dtype == torch.float32), epi, stream_of(out)))
    return out


def qk_norm_rope(qkv: torch.Tensor, heads: int, kv_heads: int, q_norm: torch.Tensor, k_norm: torch.Tensor,
                 eps: float, cos_row: torch.Tensor, sin_row: torch.Tensor, q_out: torch.Tensor,
                 k_dst: torch.Tensor, v_dst: torch.Tensor) -> None:
    """q / k per-head RMSNorm + RoPE and the K / V append (zkv_qk_norm_rope):
    qkv [bs, (heads + 2 kv_heads) * 128] bf16 -> q_out [bs, heads, 128] (any
    view with contiguous heads), k_dst / v_dst [bs, kv_heads, 128] views (the
    cache rows)."""
    from ._lib import check, lib, stream_of
    bs = qkv.shape[0]
    assert qkv.stride(1) == 1 and q_out.is_contiguous() and q_out.numel() == bs * heads * 128
    assert k_dst.shape == v_dst.shape == (bs, kv_heads, 128) and k_dst.stride(2) == v_dst.stride(2) == 1
    assert cos_row.dtype == sin_row.dtype == torch.float32 and cos_row.is_contiguous() and sin_row.is_contiguous()
    check(lib().zkv_qk_norm_rope(qkv.data_ptr(), qkv.stride(0), bs, heads, kv_heads, q_norm.data_ptr(),
                                 k_norm.data_ptr(), float(eps), cos_row.data_ptr(), sin_row.data_ptr(),
                                 q_out.data_ptr(), k_dst.data_ptr(), k_dst.stride(0), k_dst.stride(1),
                                 v_dst.data_ptr(), v_dst.stride(0), v_dst.stride(1), stream_of(qkv)))


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim in fp32, weight applied in fp32, result in x's dtype."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * weight.float()).to(x.dtype)


class RandomQwen3:
    """Random-init bf16 weights of a Qwen3 decoder (std 0.02, norms at 1), on one GPU."""

    def __init__(self, geo: Qwen3Geometry, device, seed: int = 42, max_position: int = 1 << 17,
                 fused: bool = True):
        self.geo = geo
        self.device = torch.device(device)
        self.fused = fused  # on the GPU: the fused kernels (False: the torch ops, for checks)
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)
        bf = dict(dtype=torch.bfloat16, device=self.device)

        def w(*shape):
            return (torch.randn(*shape, generator=g, device=self.device) * 0.02).to(torch.bfloat16)

        qd, kd = geo.heads * geo.head_dim, geo.kv_heads * geo.head_dim
        self.embed = w(geo.vocab, geo.hidden)             # tied with the LM head
        self.final_norm = torch.ones(geo.hidden, **bf)
        self.layers = []
        for _ in range(geo.layers):
            self.layers.append({
                "input_ln": torch.ones(geo.hidden, **bf),
                "post_ln": torch.ones(geo.hidden, **bf),
                "wqkv": w(qd + 2 * kd, geo.hidden),
                "q_norm": torch.ones(geo.head_dim, **bf),
                "k_norm": torch.ones(geo.head_dim, **bf),
                "wo": w(geo.hidden, qd),
                "gate_up": w(2 * geo.ffn, geo.hidden),
                "down": w(geo.hidden, geo.ffn),
            })
        # RoPE cos / sin (rotate-half form), fp32 [max_position, head_dim / 2]
        inv = 1.0 / (geo.rope_theta ** (torch.arange(0, geo.head_dim, 2, dtype=torch.float32,
                                                     device=self.device) / geo.head_dim))
        t = torch.arange(max_position, dtype=torch.float32, device=self.device)
        freqs = torch.outer(t, inv)
        self.cos, self.sin = freqs.cos(), freqs.sin()

    def parameter_bytes(self) -> int:
        n = self.embed.numel() + self.final_norm.numel()
        for L in self.layers:
            n += sum(t.numel() for t in L.values())
        return 2 * n

    def _rope(self, x: torch.Tensor, pos: int) -> torch.Tensor:
        """x [bs, 1, heads, 128] rotated at position pos (rotate-half, as the
        reference's fp32 path and flashinfer's is_neox=True)."""
        h = self.geo.head_dim // 2
        cos, sin = self.cos[pos], self.sin[pos]
        xf = x.float()
        x1, x2 = xf[..., :h], xf[..., h:]
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

    def layer_decode(self, ldx: int, hidden: torch.Tensor, cache) -> torch.Tensor:
        """One layer of one decode token (LLM.py:208-251); hidden [bs, 1, hidden]."""
        if hidden.is_cuda and self.fused:
            return self.layer_decode_fused(ldx, hidden, cache)
        return self.layer_decode_torch(ldx, hidden, cache)

    def layer_decode_fused(self, ldx: int, hidden: torch.Tensor, cache) -> torch.Tensor:
        """layer_decode in five kernels around cache.compute (see the module docstring)."""
        geo, L = self.geo, self.layers[ldx]
        bs = hidden.shape[0]
        qd, kd = geo.heads * geo.head_dim, geo.kv_heads * geo.head_dim
        x = hidden.reshape(bs, geo.hidden)
        qkv = torch.empty(bs, qd + 2 * kd, dtype=torch.bfloat16, device=hidden.device)
        decode_linear(x, L["wqkv"], qkv, norm_w=L["input_ln"], eps=geo.eps)
        pos = cache.context
        row = cache.decode_reserve_row(ldx)
        q = torch.empty(bs, 1, geo.heads, geo.head_dim, dtype=torch.bfloat16, device=hidden.device)
        qk_norm_rope(qkv, geo.heads, geo.kv_heads, L["q_norm"], L["k_norm"], geo.eps, self.cos[pos],
                     self.sin[pos], q, cache.unified_keys[ldx][:, :, row], cache.unified_values[ldx][:, :, row])
        attn = cache.compute(q, ldx)                                   # [bs, 1, heads, 128]
        h1 = torch.empty(bs, geo.hidden, dtype=torch.bfloat16, device=hidden.device)
        decode_linear(attn.reshape(bs, qd), L["wo"], h1, residual=x)
        act = torch.empty(bs, geo.ffn, dtype=torch.bfloat16, device=hidden.device)
        decode_linear(h1, L["gate_up"], act, norm_w=L["post_ln"], eps=geo.eps, silu_mul=True)
        h2 = torch.empty(bs, geo.hidden, dtype=torch.bfloat16, device=hidden.device)
        decode_linear(act, L["down"], h2, residual=h1)
        return h2.view(bs, 1, geo.hidden)

    def layer_decode_torch(self, ldx: int, hidden: torch.Tensor, cache) -> torch.Tensor:
        """layer_decode op by op in torch (the CPU path, and the fused path's check)."""
        geo, L = self.geo, self.layers[ldx]
        bs = hidden.shape[0]
        residual = hidden
        x = rms_norm(hidden, L["input_ln"], geo.eps)
        qkv = F.linear(x, L["wqkv"])
        qd, kd = geo.heads * geo.head_dim, geo.kv_heads * geo.head_dim
        q, k, v = qkv.split([qd, kd, kd], dim=-1)
        q = rms_norm(q.reshape(bs, 1, geo.heads, geo.head_dim), L["q_norm"], geo.eps)
        k = rms_norm(k.reshape(bs, 1, geo.kv_heads, geo.head_dim), L["k_norm"], geo.eps)
        pos = cache.context
        q, k = self._rope(q, pos), self._rope(k, pos)
        v = v.reshape(bs, 1, geo.kv_heads, geo.head_dim)
        cache.decode_update_kv_cache(k, v, ldx)
        attn = cache.compute(q, ldx)                                   # [bs, 1, heads, 128]
        hidden = residual + F.linear(attn.reshape(bs, 1, qd), L["wo"])
        residual = hidden
        x = rms_norm(hidden, L["post_ln"], geo.eps)
        gate, up = F.linear(x, L["gate_up"]).chunk(2, dim=-1)
        hidden = residual + F.linear(F.silu(gate) * up, L["down"])
        return hidden

    def decode_step(self, tokens: torch.Tensor, cache) -> torch.Tensor:
        """tokens [bs] int64 -> logits [bs, vocab] (fp32)."""
        hidden = self.embed[tokens].unsqueeze(1)
        for ldx in range(self.geo.layers):
            hidden = self.layer_decode(ldx, hidden, cache)
        if hidden.is_cuda and self.fused:
            bs = hidden.shape[0]
            logits = torch.empty(bs, self.geo.vocab, dtype=torch.float32, device=hidden.device)
            return decode_linear(hidden.reshape(bs, self.geo.hidden), self.embed, logits, norm_w=self.final_norm,
                                 eps=self.geo.eps)
        hidden = rms_norm(hidden, self.final_norm, self.geo.eps)
        return F.linear(hidden[:, 0], self.embed).float()


# Candidates kept beyond the k-th by the windowed sampler, so that ties at the
# k-th value (which top-k keeps) still fall inside the window.
_SAMPLE_TIE_WINDOW = 16
_SAMPLE_HIP_MAX_WINDOW = 64   # zkv_sample_window: one wave holds the window


def sample_next_token(logits: torch.Tensor, temperature: float = 1.0, top_p: float = 0.0,
                      top_k: int = 0, generator: torch.Generator | None = None) -> torch.Tensor:
    """Sampling of LLM.py:63-139: greedy below temperature 1e-5, else
    temperature, top-k (ties at the k-th value kept), top-p (the token that
    crosses top_p kept), softmax, one multinomial draw per row.

    With top-k on, every token the two filters keep lies among the k + 16
    largest logits unless more than 16 tokens tie with the k-th, so the sort,
    softmax and cumulative sum of top-p run over that window instead of the
    vocabulary.  The draw is torch.multinomial's for one sample (q ~ Exp(1)
    over the whole row from the same generator, then the first index of the
    largest p / q), with p / q formed only at the window's tokens: the others
    have p = 0.  Same kept set and same draw as ``sample_next_token_full``;
    the probabilities agree to rounding (their sums run in another order),
    and among tokens tied at the top-p cut the kept ones follow torch.topk's
    order where the reference's follow torch.sort's (neither is specified).
    A tie group that overflows the window (checked on the device, one host
    read) takes the full path.

    A CUDA row with k + 16 <= 64 (and a vocabulary of at most 2048 / (k + 16)
    slices of 8192) runs the whole chain as one HIP launch
    (``zkv_sample_window``) after torch draws the Exp(1) row; other rows run
    the same steps as torch ops."""
    if logits.dim() == 3:
        logits = logits.squeeze(1)
    elif logits.dim() == 1:
        logits = logits.unsqueeze(0)
    if temperature < 1e-5:
        return logits.argmax(dim=-1)
    vocab = logits.size(-1)
    if top_k <= 0 or min(top_k, vocab) + _SAMPLE_TIE_WINDOW >= vocab:
        return sample_next_token_full(logits, temperature, top_p, top_k, generator)
    window = min(top_k, vocab) + _SAMPLE_TIE_WINDOW
    if logits.is_cuda and window <= _SAMPLE_HIP_MAX_WINDOW and -(-vocab // 8192) * window <= 2048:
        return _sample_window_hip(logits, temperature, top_p, min(top_k, vocab), generator)
    scaled = logits / temperature
    k = min(top_k, vocab)
    vals, idx = torch.topk(scaled, k + _SAMPLE_TIE_WINDOW, dim=-1)
    kth = vals[..., k - 1:k]
    if bool((vals[..., -1:] == kth).any()):
        return sample_next_token_full(logits, temperature, top_p, top_k, generator)
    win = vals.masked_fill(vals < kth, float("-inf"))
    if 0.0 < top_p < 1.0:
        cum = torch.cumsum(F.softmax(win, dim=-1), dim=-1)
        remove = cum > top_p
        remove[..., 1:] = remove[..., :-1].clone()
        remove[..., 0] = False
        win = win.masked_fill(remove, float("-inf"))
    probs = F.softmax(win, dim=-1)
    q = torch.empty_like(scaled).exponential_(1, generator=generator)
    ratio = probs / q.gather(-1, idx)
    best = ratio.max(dim=-1, keepdim=True)[0]
    return torch.where(ratio == best, idx, vocab).min(dim=-1)[0]


def sample_next_token_full(logits: torch.Tensor, temperature: float = 1.0, top_p: float = 0.0,
                           top_k: int = 0, generator: torch.Generator | None = None) -> torch.Tensor:
    """LLM.py:63-139 over the whole vocabulary, op for op (the check the
    windowed ``sample_next_token`` is tested against)."""
    if logits.dim() == 3:
        logits = logits.squeeze(1)
    elif logits.dim() == 1:
        logits = logits.unsqueeze(0)
    if temperature < 1e-5:
        return logits.argmax(dim=-1)
    probs = _full_probs(logits, temperature, top_p, top_k)
    return torch.multinomial(probs, num_samples=1, generator=generator).squeeze(-1)


def _full_probs(logits: torch.Tensor, temperature: float, top_p: float, top_k: int) -> torch.Tensor:
    """The probabilities LLM.py:63-139 draws from, over the whole vocabulary."""
    logits = logits / temperature
    if top_k > 0:
        top_k = min(top_k, logits.size(-1))
        logits = logits.masked_fill(logits < torch.topk(logits, top_k)[0][..., -1, None], float("-inf"))
    if 0.0 < top_p < 1.0:
        sorted_logits, sorted_idx = torch.sort(logits, descending=True, dim=-1)
        cum = torch.cumsum(F.softmax(sorted_logits, dim=-1), dim=-1)
        remove = cum > top_p
        remove[..., 1:] = remove[..., :-1].clone()
        remove[..., 0] = False
        logits = logits.masked_fill(remove.scatter(-1, sorted_idx, remove), float("-inf"))
    return F.softmax(logits, dim=-1)


_SAMPLE_WS: dict = {}


def sample_window_launch(logits: torch.Tensor, temperature: float, top_p: float, k: int,
                         expo: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """One ``zkv_sample_window`` launch over fp32 rows [bs, vocab] with the
    Exp(1) rows ``expo``: (tokens int64 [bs], overflow flags int32 [bs])."""
    from ._lib import check, lib, ptr, stream_of
    bs, vocab = logits.shape
    dev = logits.device
    window = k + _SAMPLE_TIE_WINDOW
    L = lib()
    need = L.zkv_sample_window_workspace_size(bs, vocab, window)
    key = (dev, stream_of(logits))
    ent = _SAMPLE_WS.get(key)
    if ent is None or ent[0].numel() < need:
        ent = [torch.zeros(max(need, 1 << 12), dtype=torch.uint8, device=dev), bs]
        _SAMPLE_WS[key] = ent
    elif ent[1] != bs:
        # the arrival counters sit in the first 4 bs bytes (rounded up to 256):
        # zero them for the new row count
        ent[0][:(bs * 4 + 255) // 256 * 256].zero_()
        ent[1] = bs
    ws = ent[0]
    tokens = torch.empty(bs, dtype=torch.int64, device=dev)
    flags = torch.empty(bs, dtype=torch.int32, device=dev)
    # torch scales a CUDA tensor by a Python float as a product with the fp32 reciprocal
    inv_t = float(torch.tensor(1.0, dtype=torch.float32) / torch.tensor(temperature, dtype=torch.float32))
    check(L.zkv_sample_window(ptr(logits), logits.stride(0), bs, vocab, inv_t, k, window, float(top_p),
                              ptr(expo), expo.stride(0), ptr(tokens), ptr(flags), ptr(ws), ws.numel(),
                              stream_of(logits)))
    return tokens, flags


def _sample_window_hip(logits: torch.Tensor, temperature: float, top_p: float, k: int,
                       generator: torch.Generator | None) -> torch.Tensor:
    """sample_next_token on a CUDA row: torch draws the Exp(1) row that
    torch.multinomial would draw from the generator, then one launch ranks the
    top-(k + 16) window and applies top-k, top-p, the softmax and the draw.  A
    tie group that overflows the window draws over the whole vocabulary with
    the same Exp(1) row (one host read of the per-row flags)."""
    if logits.dtype != torch.float32 or logits.stride(-1) != 1:
        logits = logits.float().contiguous()
    expo = torch.empty_like(logits).exponential_(1, generator=generator)
    tokens, flags = sample_window_launch(logits, temperature, top_p, k, expo)
    if bool(flags.cpu().any()):
        return draw_full_vocabulary(logits, temperature, top_p, k, expo)
    return tokens


def draw_full_vocabulary(logits: torch.Tensor, temperature: float, top_p: float, top_k: int,
                         expo: torch.Tensor) -> torch.Tensor:
    """torch.multinomial(probs, 1)'s draw from the Exp(1) rows ``expo``: the
    lowest index of the largest probs / expo, probs those of LLM.py:63-139."""
    ratio = _full_probs(logits, temperature, top_p, top_k) / expo
    best = ratio.max(dim=-1, keepdim=True)[0]
    vocab = logits.size(-1)
    return torch.where(ratio == best, torch.arange(vocab, device=logits.device), vocab).min(dim=-1)[0]


def build_cache(geo: Qwen3Geometry, batch: int, context: int, max_new: int, interval: int,
                full_threshold: int, device, offload: bool = False, kv_format: str = "bf16"):
    """polar_cache for `context` prompt tokens plus `max_new` generated ones,
    with the reference's production knobs.  ``offload`` picks the bf16
    retrieval zone's home: device memory (False: the 288 GB part holds it) or
    pinned host memory (True: the reference runner's enable_offload);
    ``kv_format="kivi4"`` keeps it in device memory as 4-bit K + V instead."""
    from .cache import polar_cache
    knobs = dict(PRODUCTION_CACHE_KNOBS, enable_offload=offload, kv_format=kv_format)
    return polar_cache(
        valid_start=[0] * batch, layer_num=geo.layers, batch_size=batch, max_length=context + max_new,
        num_key_value_heads=geo.kv_heads, num_heads=geo.heads, head_dim=geo.head_dim,
        dtype=torch.bfloat16, layer_mapping={str(i): str(device) for i in range(geo.layers)},
        max_new_length=max_new, core=22, nprobe=150, cache_unit_size=8, cache_cluster_num=450,
        num_gpus=1, model_size=4, dynamic_update_interval=interval, full_attention_threshold=full_threshold,
        **knobs)


def fill_cache(cache, geo: Qwen3Geometry, batch: int, context: int, seed: int, device) -> None:
    """Prefill every layer through prefill_update_kv_cache with seeded N(0, 1)
    bf16 keys / values [batch, context, kv, 128] (what a prompt of `context`
    tokens would leave; a 64K-token prefill of random weights adds nothing)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    shape = (batch, context, geo.kv_heads, geo.head_dim)
    for ldx in range(geo.layers):
        k = torch.randn(*shape, generator=g, device=device).to(torch.bfloat16)
        v = torch.randn(*shape, generator=g, device=device).to(torch.bfloat16)
        cache.prefill_update_kv_cache(None, k, v, ldx, 0)
        del k, v


def cache_footprint(cache) -> dict:
    """Bytes the cache holds, by part: device K / V rows (bf16), the 4-bit
    records (kivi4 storage), the Format R selection metadata (chunk min / max
    / centroid, 4-bit codes, valid mask) and pinned host rows."""
    nb = lambda ts: sum(t.numel() * t.element_size() for t in ts)
    parts = {
        "device_bf16_rows": nb(cache.unified_keys + cache.unified_values),
        "device_kivi4_records": nb(getattr(cache, "kivi4_groups", None) or []),
        "device_selection_metadata": nb(cache._chunk_key_min_gpu + cache._chunk_key_max_gpu +
                                         cache._chunk_key_centroid_gpu + cache.key_kivi_packed_gpu +
                                         cache._chunk_valid_mask_gpu),
        "host_pinned_rows": nb((cache.unified_keys_cpu or []) + (cache.unified_values_cpu or [])),
    }
    parts["device_total"] = parts["device_bf16_rows"] + parts["device_kivi4_records"] + \
        parts["device_selection_metadata"]
    return parts


def attention_path_bytes(cache, layer: int) -> dict:
    """Algorithmic HBM bytes of one layer's attention path (cache.compute with
    the selection running): GQA mean + Quest bounds over the chunk metadata (one launch),
    the two top-k passes, density (when the dense and sparse per-chunk top-k
    differ; with equal values ``compute`` skips it), KIVI stage 2 over the candidate chunks, the
    top-k + gather + concat, and the attention over the selected and near-zone
    rows.  The decode append (one K / V row) is included."""
    bs, kv, d = cache.batch_size, cache.kv_head, cache.head_dim
    chunk = cache.quest_chunk_size
    n_chunks, nk = cache._cached_quest_n_chunks, cache._cached_quest_nk
    units = bs * kv
    sk = cache._chunk_skipped_count[layer]
    k_final = min(cache.final_topk, nk * chunk)
    region = cache.get_region_indices(layer)
    near = cache.sink_size + region["local_len"]
    # the Quest scan forms the GQA-mean query from the query heads and stores it
    quest = units * n_chunks * (2 * d * 2 + 1 + 4) + bs * cache.num_heads * d * 2 + units * d * 2
    topk1 = units * (n_chunks * 4 + nk * 8)
    classify = max(1, min(cache.cds_dense_topk, chunk)) != max(1, min(cache.cds_sparse_topk, chunk))
    density = units * (nk * (8 + d * 2 + 4) + d * 2) if classify else 0    # skipped when dense = sparse
    topk2 = units * (nk * 4 + nk) if classify else 0
    # stage 2 writes (and the top-k reads) width lanes per chunk: the kept ones
    # when compute uses the compact output, else the whole chunk
    width = cache._stage2_out_width(layer) or chunk
    stage2 = units * (nk * (8 + 1 + 16 * chunk * 4 + 2 * d * 2) + nk * width * 12)
    gather = units * (nk * width * 12 + sk * 8 + (k_final + sk) * 8)
    if getattr(cache, "kv_format", "bf16") == "kivi4":
        # the selected tokens from 4-bit records (160 B per token per KV head:
        # K / V codes and their share of the scale / zero), the skipped tail
        # and the near zone as bf16 rows
        attn = units * (k_final * 160 + (sk + near) * 2 * d * 2 + (k_final + sk) * 8) + \
            2 * bs * cache.num_heads * d * 2
    else:
        attn = units * ((k_final + sk + near) * 2 * d * 2 + (k_final + sk) * 8) + 2 * bs * cache.num_heads * d * 2
    append = 2 * units * d * 2
    parts = {"quest_gqa": quest, "topk_chunks": topk1, "density": density,
             "topk_dense": topk2, "kivi_stage2": stage2, "topk_gather_concat": gather,
             "attention": attn, "append": append}
    parts["total"] = sum(parts.values())
    return parts
