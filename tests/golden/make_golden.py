"""Write the golden fixtures under tests/golden/ from the reference's own
pure-PyTorch functions.

Run in a container that holds the reference checkout (default
/root/reference, or $ZOOMKV_REFERENCE); the fixtures it writes are plain
npz data (inputs and expected outputs) and are what the tests read.  Nothing
at test time, on the CPU or on the GPU, imports the reference.

Reference functions called (Z/ = runtime/zoomkv_urania_runtime_20261011/):
  * Z/cache_hub/kivi/quant_pack.py      quantize_kcache_4bit, pack_kcache_4bit,
                                        unpack_kcache_4bit (:86-198)
  * Z/cache_hub/kivi/qk_dot.py          partial_chunk_kivi_qk_ref (:114-175)
  * Z/cache_hub/quest/quest_ops.py      QuestPytorch.quest_chunk_score (:22-31)
  * Z/cache_hub/lse_merge/lse_merge.py  lse_merge_torch (:79-119)
The chunk statistics and the chunk-major relayout of the packed codes are the
torch calls of S:2133-2135 and S:2017 (S = Z/cache_hub/
polar_cache_quest_density_single_layer_kivi.py), whose class cannot be built
without CUDA; they are made here with the same torch ops on the CPU.

The package initialisers of ``cache_hub`` import flash-attn, which is not
installed, so the four files are loaded by path; ``qk_dot.py`` imports
``cache_hub.kivi.quant_pack``, which is registered under that name (the real
file) beneath two empty package entries.

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import importlib.util
import os
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REF = Path(os.environ.get("ZOOMKV_REFERENCE", "/root/reference")) / "runtime" / "zoomkv_urania_runtime_20261011"
SEED = 42


def _load(name: str, rel: str):
    spec = importlib.util.spec_from_file_location(name, REF / rel)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _reference_modules():
    for pkg in ("cache_hub", "cache_hub.kivi"):
        if pkg not in sys.modules:
            m = types.ModuleType(pkg)
            m.__path__ = []
            sys.modules[pkg] = m
    qp = _load("cache_hub.kivi.quant_pack", "cache_hub/kivi/quant_pack.py")
    qk = _load("cache_hub.kivi.qk_dot", "cache_hub/kivi/qk_dot.py")
    qo = _load("zoomkv_ref_quest_ops", "cache_hub/quest/quest_ops.py")
    lm = _load("zoomkv_ref_lse_merge", "cache_hub/lse_merge/lse_merge.py")
    return qp, qk, qo, lm


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def _keys(gen: torch.Generator, bs: int, kv: int, n: int, outliers: int = 4) -> torch.Tensor:
    """N(0,1) keys with `outliers` channels scaled by 10 (the C1 shape's rule)."""
    k = torch.randn(bs, kv, n, 128, generator=gen)
    ch = torch.randperm(128, generator=gen)[:outliers]
    k[..., ch] *= 10.0
    return k.to(torch.bfloat16)


def make_kivi_quant_pack(qp, gen):
    """quant_pack.py on chunk statistics from S:2133-2135, for g in 8 / 16 / 32.

    Edge rows: channels 0..7 of head 0's first 32 tokens are flat (every chunk
    min == max there, scale 0 -> the 1e-8 divisor), and head 1's token 5 holds
    the chunk max of every channel exactly."""
    bs, kv, n = 1, 2, 64
    K = _keys(gen, bs, kv, n)
    K[0, 0, :32, :8] = K[0, 0, 0, :8]
    K[0, 1, 5, :] = K[0, 1, :8, :].amax(dim=0)
    out = {"K": bits(K)}
    for g in (8, 16, 32):
        kc = K.view(bs, kv, n // g, g, 128)
        mn, mx, mean = kc.amin(dim=3), kc.amax(dim=3), kc.mean(dim=3)
        codes = qp.quantize_kcache_4bit(K, mn, mx, g)
        packed, scale = qp.pack_kcache_4bit(K, mn, mx, g)
        deq = qp.unpack_kcache_4bit(packed, mn, mx, g)
        packed_cm = packed.view(bs, kv, n // g, g, 16).transpose(-1, -2).contiguous()   # S:2017
        out.update({
            f"g{g}_min": bits(mn), f"g{g}_max": bits(mx), f"g{g}_mean": bits(mean),
            f"g{g}_codes": codes.numpy().astype(np.uint8),
            f"g{g}_packed_cm": packed_cm.numpy(),
            f"g{g}_scale": bits(scale), f"g{g}_dequant": bits(deq),
        })
    return out


def make_kivi_qk(qp, qk, gen):
    """partial_chunk_kivi_qk_ref on a chunk-major pack, g = 16 (dense 16 /
    sparse 8) and g = 8 (dense 8 / sparse 4), 8 of 12 chunks selected."""
    out = {}
    bs, kv, nc, nk = 1, 2, 12, 8
    for g, dense, sparse in ((16, 16, 8), (8, 8, 4)):
        K = _keys(gen, bs, kv, nc * g)
        kc = K.view(bs, kv, nc, g, 128)
        mn, mx = kc.amin(dim=3), kc.amax(dim=3)
        packed, _ = qp.pack_kcache_4bit(K, mn, mx, g)
        packed_cm = packed.view(bs, kv, nc, g, 16).transpose(-1, -2).contiguous()
        q = torch.randn(bs, kv, 128, generator=gen).to(torch.bfloat16)
        ids = torch.stack([torch.randperm(nc, generator=gen)[:nk] for _ in range(bs * kv)]).view(bs, kv, nk)
        mask = torch.rand(bs, kv, nk, generator=gen) < 0.5
        s_out = torch.empty(bs, kv, nk * g, dtype=torch.float32)
        i_out = torch.empty(bs, kv, nk * g, dtype=torch.int64)
        qk.partial_chunk_kivi_qk_ref(ids, mask, packed_cm, mn, mx, q, group_size=g, dense_topk=dense,
                                     sparse_topk=sparse, out_scores=s_out, out_indices=i_out)
        out.update({
            f"g{g}_packed_cm": packed_cm.numpy(), f"g{g}_min": bits(mn), f"g{g}_max": bits(mx),
            f"g{g}_raw_q": bits(q), f"g{g}_chunk_ids": ids.numpy(), f"g{g}_dense_mask": mask.numpy(),
            f"g{g}_topk": np.array([dense, sparse], dtype=np.int32),
            f"g{g}_scores": s_out.numpy(), f"g{g}_indices": i_out.numpy(),
        })
    return out


def make_quest(qo, gen):
    """QuestPytorch.quest_chunk_score over bf16 chunk min / max of real keys,
    37 of 40 chunks scored, some chunks invalid."""
    bs, kv, nmax, n, g = 2, 2, 40, 37, 16
    K = _keys(gen, bs, kv, nmax * g)
    kc = K.view(bs, kv, nmax, g, 128)
    mn, mx = kc.amin(dim=3), kc.amax(dim=3)
    q = torch.randn(bs, kv, 128, generator=gen).to(torch.bfloat16)
    valid = torch.rand(bs, kv, nmax, generator=gen) < 0.85
    scores = torch.empty(bs, kv, n, dtype=torch.float32)
    qo.QuestPytorch().quest_chunk_score(q, mn, mx, scores, n, valid)
    return {"raw_q": bits(q), "chunk_min": bits(mn), "chunk_max": bits(mx), "valid": valid.numpy(),
            "n_chunks": np.array(n, dtype=np.int32), "scores": scores.numpy()}


def make_lse_merge(lm, gen):
    """lse_merge_torch on fp32 and bf16 partials; lse in the flash-attn
    [bs, heads, 1] layout, one pair far apart (weight underflow side)."""
    bs, h, d = 2, 8, 128
    a = torch.randn(bs, 1, h, d, generator=gen)
    b = torch.randn(bs, 1, h, d, generator=gen)
    la = torch.randn(bs, h, 1, generator=gen) * 3.0
    lb = torch.randn(bs, h, 1, generator=gen) * 3.0
    lb[0, 0, 0] = la[0, 0, 0] + 40.0
    out = {"a": a.numpy(), "b": b.numpy(), "lse_a": la.numpy(), "lse_b": lb.numpy(),
           "merged_f32": lm.lse_merge_torch(a, la, b, lb).numpy()}
    ab, bb = a.to(torch.bfloat16), b.to(torch.bfloat16)
    out.update({"a_bf16": bits(ab), "b_bf16": bits(bb),
                "merged_bf16": bits(lm.lse_merge_torch(ab, la, bb, lb))})
    return out


def main() -> None:
    torch.set_num_threads(1)
    qp, qk, qo, lm = _reference_modules()
    gen = torch.Generator().manual_seed(SEED)
    fixtures = {
        "kivi_quant_pack": make_kivi_quant_pack(qp, gen),
        "kivi_qk_ref": make_kivi_qk(qp, qk, gen),
        "quest_torch": make_quest(qo, gen),
        "lse_merge_torch": make_lse_merge(lm, gen),
    }
    for name, arrays in fixtures.items():
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **arrays)
        print(f"wrote {path.relative_to(HERE.parent.parent)} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
