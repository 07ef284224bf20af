"""Shared helpers for the KV data-path tests (numpy <-> torch bit patterns)."""
from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"

TORCH_DTYPE = {"bf16": "bfloat16", "fp16": "float16"}


def tdtype(name: str):
    import torch
    return getattr(torch, TORCH_DTYPE[name])


def to_device_bits(bits: np.ndarray, dtype: str, device):
    """uint16 bit patterns -> GPU tensor of the 16-bit float dtype."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16))
    return t.view(tdtype(dtype)).to(device)


def to_bits(t) -> np.ndarray:
    """16-bit float tensor -> uint16 numpy bit patterns (copied to host)."""
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def random_bits(rng: np.random.Generator, shape, dtype: str) -> np.ndarray:
    """N(0,1) values cast (round-to-nearest-even) to bf16/fp16 bit patterns."""
    x = rng.standard_normal(shape).astype(np.float32)
    if dtype == "fp16":
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def load_golden(name: str = "cfg1_tiny.npz"):
    return np.load(GOLDEN / name, allow_pickle=False)


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (8 significant bits)."""
    ax = np.maximum(np.abs(x), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


def fp16_ulp(x: np.ndarray) -> np.ndarray:
    ax = np.maximum(np.abs(x), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(ax)) - 10)
