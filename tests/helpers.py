"""Shared helpers for tests: dtype conversions between torch and the oracle's
numpy bit patterns, and seeded synthetic inputs."""

from __future__ import annotations

import numpy as np
import torch

TORCH_DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def to_bits(t: torch.Tensor) -> np.ndarray:
    """torch tensor -> numpy storage the oracle takes (uint16 bits or f32)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.numpy().copy()


def from_bits(a: np.ndarray, dtype: str) -> torch.Tensor:
    if dtype == "f32":
        return torch.from_numpy(np.ascontiguousarray(a, np.float32))
    t = torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16))
    return t.view(TORCH_DT[dtype])


def same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    a = a.detach().cpu().contiguous()
    b = b.detach().cpu().contiguous()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.dtype.is_floating_point:
        width = {2: torch.int16, 4: torch.int32, 8: torch.int64}[a.element_size()]
        return torch.equal(a.view(width), b.view(width))
    return torch.equal(a, b)


def randn(shape, dtype: str, seed: int, scale: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(TORCH_DT[dtype])


def minmax_pages(dtype: str, G: int, P: int, D: int, seed: int):
    """lo = min(a, b), hi = max(a, b) as in scripts/test_twilight_fused_quest_v1.py:17-19."""
    a = randn((G, P, D), dtype, seed)
    b = randn((G, P, D), dtype, seed + 1)
    return torch.minimum(a, b), torch.maximum(a, b)
