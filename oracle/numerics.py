"""Explicit IEEE rounding helpers for the oracle (test infrastructure only).

bfloat16 values are carried as float32 arrays whose low 16 mantissa bits are
zero; storage / comparison uses the uint16 bit pattern.  float16 values use
numpy's float16, whose float32->float16 cast is round-to-nearest-even
including subnormals.
"""
from __future__ import annotations

import numpy as np


def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit pattern, round-to-nearest-even (NaN kept quiet)."""
    u = f32(x).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    bias = ((u >> 16) & 1) + 0x7FFF
    r = ((u + bias) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16r(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (RNE); result as float32."""
    return bf16_to_f32(bf16_bits(x))


def f16_bits(x) -> np.ndarray:
    """float32 -> float16 bit pattern (RNE, numpy semantics)."""
    return f32(x).astype(np.float16).view(np.uint16)


def f16_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# torch's clamp(min=1e-8) on a bfloat16 tensor compares against the scalar
# converted to the tensor dtype (S:2006, quant_pack.py:116).
BF16_1EM8 = bf16r(np.float32(1e-8))


def random_bf16(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    """Seeded N(0, scale^2) values rounded to bfloat16 (as float32)."""
    return bf16r(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))
