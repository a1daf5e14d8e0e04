"""Shared test helpers: seeded inputs and numpy <-> torch conversion."""
from __future__ import annotations

import numpy as np
import torch

from oracle.numerics import bf16r


def gaussian_bf16(rng, shape, outlier_channels=0, outlier_scale=10.0):
    """N(0,1) bf16 values; ``outlier_channels`` channels of the last dim x scale."""
    x = rng.standard_normal(shape, dtype=np.float32)
    if outlier_channels:
        ch = rng.permutation(shape[-1])[:outlier_channels]
        x[..., ch] *= np.float32(outlier_scale)
    return bf16r(x)


def to_bf16(x: np.ndarray, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(device=device, dtype=torch.bfloat16)


def from_torch(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.float().cpu().numpy()
    if t.dtype == torch.float16:
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()
