"""Write tests/golden/rabitq4_pariskv.npz from the reference's own ParisKV
4-bit RaBitQ code (pure PyTorch, run on the CPU).

Run in a container that holds the reference checkout (default
/root/reference, or $ZOOMKV_REFERENCE).  The fixture is plain npz data
(inputs and expected outputs); nothing at test time imports the reference.

Reference code executed (P/ = runtime/pariskv_urania_runtime_20261011/):
  * P/cache_hub/polar_cache.py  ``batch_encode`` (:1130-1195),
    ``_pack_4bit_codes`` (:1067-1084) and ``_encode_query_blocks``
    (:1108-1124), methods of the ParisKV cache class.  The class cannot be
    built without CUDA and the module's imports (flash-attn) are absent, so
    the three method bodies are compiled from the file's own text (``ast``)
    and bound to an object holding the attributes the constructor sets:
    ``quantizer.srht_diagonal_signs`` (PC:79-93; a seeded +-1 vector here,
    passed in as input), ``_hadamard_scale`` (PC:428), ``_mag_thresholds`` /
    ``_mag_centers`` (PC:266-270, read from the file as numbers) and
    ``_bitpack_shifts`` (PC:273).  ``hadamard_transform`` is the reference's
    fallback, P/cache_hub/hadamard_fallback.py.
  * P/cache_hub/rerank/rerank.py ``_unpack_4bit_codes`` (:165-186).
  * P/cache_hub/rerank/test_rerank_topk.py ``python_rabitq_scores``
    (:60-113): the reference test's sequential-bf16 model of the rerank
    kernel rerank.cu:52-143, which that test requires to equal the kernel
    bit for bit.

Usage: python tests/golden/make_golden_rabitq4.py
"""
from __future__ import annotations

import ast
import importlib.util
import os
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REF = Path(os.environ.get("ZOOMKV_REFERENCE", "/root/reference")) / "runtime" / "pariskv_urania_runtime_20261011"
SEED = 7


def _load(name: str, path: Path):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _methods(path: Path, names):
    """The named methods of polar_cache.py, compiled from its own text."""
    tree = ast.parse(path.read_text())
    found = {}
    consts = {}
    for node in ast.walk(tree):
        if isinstance(node, ast.FunctionDef) and node.name in names and node.name not in found:
            found[node.name] = node
        if isinstance(node, ast.Assign) and len(node.targets) == 1 and isinstance(node.targets[0], ast.Name):
            if node.targets[0].id == "DEFAULT_SRHT_ROUNDS":
                consts["DEFAULT_SRHT_ROUNDS"] = ast.literal_eval(node.value)
    return found, consts


def _levels(path: Path):
    """The literal lists of ``_mag_thresholds`` / ``_mag_centers`` (PC:266-270)."""
    tree = ast.parse(path.read_text())
    out = {}
    for node in ast.walk(tree):
        if isinstance(node, ast.Assign) and len(node.targets) == 1 and isinstance(node.targets[0], ast.Attribute):
            attr = node.targets[0].attr
            if attr in ("_mag_thresholds", "_mag_centers") and attr not in out:
                call = node.value  # torch.tensor([...], ...).contiguous()
                while not call.args:
                    call = call.func.value
                out[attr] = ast.literal_eval(call.args[0])
    return out


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main() -> None:
    pc = REF / "cache_hub" / "polar_cache.py"
    hf = _load("pariskv_hadamard_fallback", REF / "cache_hub" / "hadamard_fallback.py")
    rr = _load("rerank", REF / "cache_hub" / "rerank" / "rerank.py")
    tr = _load("pariskv_test_rerank_topk", REF / "cache_hub" / "rerank" / "test_rerank_topk.py")
    fns, consts = _methods(pc, {"batch_encode", "_pack_4bit_codes", "_encode_query_blocks"})
    lv = _levels(pc)
    ns = {"torch": torch, "hadamard_transform": hf.hadamard_transform, **consts}
    mod = ast.Module(body=list(fns.values()), type_ignores=[])
    exec(compile(ast.fix_missing_locations(mod), str(pc), "exec"), ns)

    gen = torch.Generator().manual_seed(SEED)
    signs = (torch.randint(0, 2, (128,), generator=gen) * 2 - 1).to(torch.bfloat16)
    obj = types.SimpleNamespace()
    obj.quantizer = types.SimpleNamespace(srht_diagonal_signs=[signs] * consts["DEFAULT_SRHT_ROUNDS"], B=16, m=8)
    obj._hadamard_scale = 1.0 / np.sqrt(128)
    obj._mag_thresholds = torch.tensor(lv["_mag_thresholds"], dtype=torch.bfloat16)
    obj._mag_centers = torch.tensor(lv["_mag_centers"], dtype=torch.bfloat16)
    obj._bitpack_shifts = 1 << torch.arange(8, dtype=torch.uint8)
    obj.polar_B, obj.polar_m = 16, 8
    for name in ("batch_encode", "_pack_4bit_codes", "_encode_query_blocks"):
        setattr(obj, name, types.MethodType(ns[name], obj))

    # keys: N(0,1) with outlier channels, plus edge rows: a zero key, a key
    # of 1e-6 entries, a key of 3000s, one block of zeros, repeated rows
    bs, kv, n = 1, 2, 300
    K = torch.randn(bs, kv, n, 128, generator=gen)
    K[..., torch.randperm(128, generator=gen)[:4]] *= 10.0
    K[0, 0, 0] = 0.0
    K[0, 0, 1] = 1e-6
    K[0, 1, 2] = 3000.0 * torch.sign(torch.randn(128, generator=gen))
    K[0, 1, 3, 40:48] = 0.0
    K[0, 1, 4] = K[0, 1, 5]
    K = K.to(torch.bfloat16)
    codebook, weight, packed = obj.batch_encode(K)
    q = torch.randn(bs, kv, 128, generator=gen).to(torch.bfloat16)
    q_blocks, q_norm = obj._encode_query_blocks(q)

    s_sign, t_codes = rr._unpack_4bit_codes(packed.reshape(-1, 4), m=8)

    # rerank: candidate lists (sorted and unsorted, repeats) per (b, kv)
    cand = torch.stack([torch.randperm(n, generator=gen)[:96] for _ in range(bs * kv)]).view(bs, kv, 96)
    cand[0, 0, :4] = torch.tensor([0, 1, 0, n - 1])
    # the test's q_norm is [bs, kv] (test_rerank_topk.py:50); the cache's is [bs, kv, 1]
    scores = tr.python_rabitq_scores(cand, packed, weight, q_blocks, q_norm.squeeze(-1), obj._mag_centers, 16, 8)

    out = {
        "signs": bits(signs), "keys": bits(K), "codebook": codebook.numpy(), "block_weight": bits(weight),
        "packed_4bit": packed.numpy(), "q": bits(q), "q_blocks": bits(q_blocks), "q_norm": bits(q_norm),
        "unpack_sign": s_sign.numpy().reshape(packed.shape[:-1] + (8,)),
        "unpack_t": t_codes.numpy().astype(np.uint8).reshape(packed.shape[:-1] + (8,)),
        "cand": cand.numpy(), "scores": bits(scores),
        "mag_thresholds": bits(obj._mag_thresholds), "mag_centers": bits(obj._mag_centers),
    }
    path = HERE / "rabitq4_pariskv.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes): " + ", ".join(f"{k}{list(v.shape)}" for k, v in out.items()))


if __name__ == "__main__":
    main()
