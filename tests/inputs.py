"""Seeded synthetic inputs shared by the CPU and GPU tests (bf16 bits generated on the CPU so that
both sides see identical values).  Generator seed = 20250101 + config index, as the benchmark uses."""

from __future__ import annotations

import math

import numpy as np
import torch

SEED0 = 20250101


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def randn_bf16(shape, gen, std=1.0):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(torch.bfloat16)


def qkv(B, Lq, Lk, Hq, Hkv, D=128, seed=SEED0, k_offset_std=0.0, dtype=torch.bfloat16):
    """q, k, v ~ N(0, 1) in NHD; k gets a per-(head, channel) offset ~ N(0, k_offset_std)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, Lq, Hq, D), generator=g, dtype=torch.float32)
    k = torch.randn((B, Lk, Hkv, D), generator=g, dtype=torch.float32)
    v = torch.randn((B, Lk, Hkv, D), generator=g, dtype=torch.float32)
    if k_offset_std:
        k = k + torch.randn((1, 1, Hkv, D), generator=g, dtype=torch.float32) * k_offset_std
    return q.to(dtype), k.to(dtype), v.to(dtype)


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (math.sqrt(a @ a) * math.sqrt(b @ b) + 1e-300))
