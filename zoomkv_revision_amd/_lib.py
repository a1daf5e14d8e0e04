"""ctypes binding of libzoomkv_gfx950.so (the C ABI declared in include/zoomkv_gfx950.h).

There is no fallback: if the library is missing or fails to load, every op
raises.  Errors returned by an entry point become ``RuntimeError`` carrying
``zkv_last_error()``, mirroring the reference's TORCH_CHECK -> RuntimeError
convention (e.g. Z/cache_hub/kivi/kivi_qk_dot.cu:338-394).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("ZOOMKV_GFX950_LIB",
                               Path(__file__).resolve().parent / "libzoomkv_gfx950.so"))

P = C.c_void_p
I32 = C.c_int
I64 = C.c_int64
F32 = C.c_float
SZ = C.c_size_t

# name -> (restype, argtypes); kept in the order of include/zoomkv_gfx950.h
SIGNATURES = {
    "zkv_last_error": (C.c_char_p, []),
    "zkv_version": (C.c_char_p, []),
    "zkv_chunk_encode": (I32, [P, I64, I64, I64, I32, I32, I32, I32, I32, I32,
                               P, P, P, P, P, P]),
    "zkv_kivi4_pack": (I32, [P, I64, I64, I64, P, I64, I64, I64, I32, I32, I32, I32, I32,
                             P, P, P]),
    "zkv_kivi4_prefill": (I32, [P, I64, I64, I64, P, I64, I64, I64, I32, I32, I32, I32, I32,
                                P, P, P, P, I32, I32, I32, P]),
    "zkv_kivi4_attention_workspace_size": (SZ, [I32, I32, I32, I32, I32, I32]),
    "zkv_kivi4_decode_attention": (I32, [P, I64, I64, P, I32, P, P, I32,
                                         I32, I32, I32, I32, I32, F32, P, I32, P, I32,
                                         P, SZ, P]),
    "zkv_kivi4_decode_attention_noalloc": (I32, [P, I64, I64, P, I32, P, P, I32,
                                                 I32, I32, I32, I32, I32, F32, P, I32, P, I32, P]),
    "zkv_kivi4_attention_partial": (I32, [P, I64, I64, P, I32, P, P, I32,
                                          I32, I32, I32, I32, I32, F32, I32, P, SZ, P, P]),
    "zkv_attention_merge": (I32, [P, I32, I32, I32, I32, P, I32, P]),
    "zkv_quest_chunk_score": (I32, [P, P, P, I32, P, I32, I32, I32, I32, P, P]),
    "zkv_quest_chunk_score_gqa": (I32, [P, I64, I64, I32, P, P, P, I32, P, I32, I32, I32, I32, P, P]),
    "zkv_quest_chunk_topk_gqa": (I32, [P, I64, I64, I32, P, P, P, I32, P, I32, I32, I32, I32, P, I32, P, I64,
                                       P, SZ, P]),
    "zkv_topk": (I32, [P, I64, I32, I32, I32, P, I64, P, I64, P, I64, I32, I64, P]),
    "zkv_chunk_density_scores": (I32, [P, I64, I64, P, I64, I64, I64, P, I64, I64, P, I64, I64,
                                       I32, I32, I32, I32, P]),
    "zkv_dense_mask_from_topk": (I32, [P, P, I32, I32, I32, P]),
    "zkv_topk_dense_mask": (I32, [P, I64, I32, I32, I32, P, I64, P, I64, P]),
    "zkv_gqa_mean_query": (I32, [P, I64, I64, I32, I32, I32, P, P]),
    "zkv_kivi_qk_dense_sparse": (I32, [P, I64, I64, P, I64, I64, P, I64, I64, I32, P, P, I64, I64,
                                       I32, P, I64, I64, I32, I32, I32, P, P, I64, I64,
                                       I32, I32, I32, P]),
    "zkv_kivi_qk_dense_sparse_compact": (I32, [P, I64, I64, P, I64, I64, P, I64, I64, I32, P, P, I64, I64,
                                               I32, P, I64, I64, I32, I32, I32, I32, P, P, I64, I64,
                                               I32, I32, I32, P]),
    "zkv_page_minmax_f16": (I32, [P, I64, I64, I64, I32, I32, I32, I32, I32, P, P, P]),
    "zkv_kivi4_sparse_attention_workspace_size": (SZ, [I32, I32, I32, I32, I32, I32]),
    "zkv_kivi4_sparse_attention": (I32, [P, I64, I64, P, I32, P, P, I32, I32, I32, I32, I32,
                                         I32, P, I64, I64, I32, F32, P, I32, P, I32, P, SZ, P]),
    "zkv_kivi4_token_attention_workspace_size": (SZ, [I32, I32, I32, I32, I32, I32]),
    "zkv_kivi4_token_attention": (I32, [P, I64, I64, P, I32, I32, P, I64, I64, I64, P, I64, I64, I64, I32,
                                        P, I64, I64, I32, I32, I32, I32, I32, I32, I32, I32, F32, P, I32, P, I32,
                                        P, SZ, P]),
    "zkv_bf16_attention_workspace_size": (SZ, [I32, I32, I32, I32, I32]),
    "zkv_bf16_decode_attention": (I32, [P, I64, I64, P, I64, I64, I64, P, I64, I64, I64, I32, I32, I32, I32,
                                        F32, P, I32, P, I32, P, SZ, P]),
    "zkv_bf16_gather_attention": (I32, [P, I64, I64, P, I64, I64, I64, P, I64, I64, I64, I32, P, I64, I64,
                                        I32, I32, I32, I32, I32, I32, F32, P, I32, P, I32, P, SZ, P]),
    "zkv_lse_merge": (I32, [P, P, P, P, P, I32, I32, I32, I32, P]),
    "zkv_rabitq_encode": (I32, [P, I64, I64, P, P, P, P]),
    "zkv_rabitq_estimate": (I32, [P, P, P, P, I32, I32, I64, P, P]),
    "zkv_rabitq_search_workspace_size": (SZ, [I32, I32, I64, I32]),
    "zkv_rabitq_search": (I32, [P, P, I64, I64, P, P, P, I32, I32, I64, I32, P, P, P, P, SZ, P]),
    "zkv_rabitq4_encode": (I32, [P, I64, I64, I64, I32, I32, I32, P, P, P, P, I64, I64, I64, P, I64, I64, I64,
                                 P, I64, I64, I64, I32, P]),
    "zkv_rabitq4_encode_query": (I32, [P, I64, I32, P, P, P, P]),
    "zkv_rabitq4_rerank": (I32, [P, I64, I64, I32, I32, I32, P, I64, I64, I64, I64, I32, P, I64, I64, I64,
                                 P, P, P, P, P, P, P, SZ, P]),
    "zkv_rabitq4_rerank_workspace_size": (SZ, [I32, I32, I32]),
    "zkv_h2d_gather_kv": (I32, [P, P, I32, I32, I32, P, I32, P, P, I32, P]),
    "zkv_h2d_gather_kv_packed": (I32, [P, P, I32, I32, I32, P, P, I64, P, I64, P, P, I32, I32, P]),
    "zkv_copy_rows": (I32, [P, SZ, P, SZ, SZ, SZ, P]),
    "zkv_host_alloc": (I32, [SZ, P]),
    "zkv_host_free": (I32, [P]),
    "zkv_decode_linear": (I32, [P, I64, I32, I32, P, I32, P, F32, P, I64, P, I64, I32, I32, P]),
    "zkv_qk_norm_rope": (I32, [P, I64, I32, I32, I32, P, P, F32, P, P, P, P, I64, I64, P, I64, I64, P]),
    "zkv_sample_window_workspace_size": (SZ, [I32, I32, I32]),
    "zkv_sample_window": (I32, [P, I64, I32, I32, F32, I32, I32, F32, P, I64, P, P, P, SZ, P]),
}

_lib = None


class ZkvError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """Load (once) and return the native library; raise if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ZkvError(
                f"libzoomkv_gfx950.so not found at {LIB_PATH}; build it with "
                "`python -m zoomkv_revision_amd.build` (no CPU fallback exists)")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().zkv_last_error().decode(errors="replace")
        raise ZkvError(f"zoomkv_gfx950 error {rc}: {msg}")


_raw_stream = torch._C._cuda_getCurrentRawStream


def device_stream(device: torch.device) -> int:
    """The raw handle of the current stream of a torch device."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return _raw_stream(idx)


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of t's device (what the reference's kernels use),
    as its raw handle (no Stream object is built per call)."""
    return _raw_stream(t.get_device())


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ZkvError("zoomkv_gfx950 ops take device tensors (no CPU path exists)")
