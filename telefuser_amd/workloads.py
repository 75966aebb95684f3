"""Synthetic inputs of the benchmark configurations (shapes from the Wan2.1 / LingBot call sites).

Inputs are generated with a seeded torch.Generator (seed = 20250101 + config index [+ call index]).
Config 2 follows the Wan self-attention prologue (telefuser/models/wan_video_dit.py:192-207):
q, k = RMSNorm over the full hidden size (weight 1, eps 1e-6) then interleaved 3-D RoPE with the
f/h/w frequency split D - 2*(D//3), D//3, D//3 (wan_video_dit.py:60-65) over the latent grid.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

SEED0 = 20250101


@dataclass(frozen=True)
class AttnConfig:
    name: str
    B: int
    Lq: int
    Lk: int
    Hq: int
    Hkv: int
    D: int = 128
    grid: tuple | None = None  # (f, h, w) latent grid for RoPE, or None
    k_offset_std: float = 0.0
    pad_range: tuple | None = None  # key padding drawn from [lo, hi] (config 4)
    index: int = 0

    def ops(self) -> float:
        """Algorithmic work per call: 4 * B * Hq * Lq * Lk * D (QK^T + PV, no causal discount)."""
        return 4.0 * self.B * self.Hq * self.Lq * self.Lk * self.D


CONFIGS = {
    "c1": AttnConfig("c1_cpu_op", 1, 1024, 1024, 2, 2, k_offset_std=0.5, index=0),
    "c2": AttnConfig("wan2.1-1.3b_480p_self_attn", 1, 32760, 32760, 12, 12, grid=(21, 30, 52), index=1),
    "c3": AttnConfig("wan2.1-14b_720p_self_attn", 1, 75600, 75600, 40, 40, k_offset_std=1.0, index=2),
    "c4": AttnConfig("wan2.1-14b_text_cross_attn", 1, 75600, 512, 40, 40, pad_range=(100, 300), index=3),
    "c5": AttnConfig("lingbot_stream_chunk_vs_kv_cache", 1, 4680, 32760, 12, 12, index=4),
}


def _rope_3d(x: torch.Tensor, grid: tuple) -> torch.Tensor:
    """Interleaved-pair RoPE with per-axis frequencies over a (f, h, w) grid.  x: [B, L, H, D] fp32."""
    B, L, H, D = x.shape
    f, h, w = grid
    dims = (D - 2 * (D // 3), D // 3, D // 3)
    angles = []
    pos = torch.stack(torch.meshgrid(torch.arange(f), torch.arange(h), torch.arange(w), indexing="ij"), -1)
    pos = pos.reshape(-1, 3)[:L].to(x.device, torch.float64)
    for axis, d in enumerate(dims):
        freqs = 1.0 / (10000.0 ** (torch.arange(0, d, 2, device=x.device, dtype=torch.float64)[: d // 2] / d))
        angles.append(torch.outer(pos[:, axis], freqs))
    ang = torch.cat(angles, dim=1)  # [L, D/2]
    cos, sin = ang.cos().float()[None, :, None, :], ang.sin().float()[None, :, None, :]
    xr = x.reshape(B, L, H, D // 2, 2)
    a, b = xr[..., 0], xr[..., 1]
    return torch.stack((a * cos - b * sin, a * sin + b * cos), dim=-1).reshape(B, L, H, D)


def make_inputs(cfg: AttnConfig, device, call: int = 0, dtype=torch.bfloat16):
    """q [B, Lq, Hq, D], k/v [B, Lk, Hkv, D] in NHD, plus kv_valid_len (list or None)."""
    g = torch.Generator(device=device).manual_seed(SEED0 + cfg.index + 1000 * call)
    q = torch.randn((cfg.B, cfg.Lq, cfg.Hq, cfg.D), generator=g, device=device, dtype=torch.float32)
    k = torch.randn((cfg.B, cfg.Lk, cfg.Hkv, cfg.D), generator=g, device=device, dtype=torch.float32)
    v = torch.randn((cfg.B, cfg.Lk, cfg.Hkv, cfg.D), generator=g, device=device, dtype=torch.float32)
    if cfg.k_offset_std:
        k += torch.randn((1, 1, cfg.Hkv, cfg.D), generator=g, device=device) * cfg.k_offset_std
    if cfg.grid is not None:
        def norm(x):
            flat = x.reshape(cfg.B, x.shape[1], -1)
            flat = flat * torch.rsqrt(flat.pow(2).mean(-1, keepdim=True) + 1e-6)
            return flat.reshape(x.shape)
        q = _rope_3d(norm(q), cfg.grid)
        k = _rope_3d(norm(k), cfg.grid)
    kv_valid = None
    if cfg.pad_range is not None:
        lo, hi = cfg.pad_range
        pads = torch.randint(lo, hi + 1, (cfg.B,), generator=torch.Generator().manual_seed(SEED0 + cfg.index))
        kv_valid = [cfg.Lk - int(p) for p in pads]
        for bi, n in enumerate(kv_valid):
            k[bi, n:] = 0
            v[bi, n:] = 0
    return q.to(dtype), k.to(dtype), v.to(dtype), kv_valid


def peak_ops(pv: str = "fp8") -> float:
    """MI355X dense MFMA peak for the mix: INT8 QK (5.0 POPS) + FP8 PV (5.0 PFLOPS); with bf16 PV
    (2.5 PFLOPS) the equal-work harmonic mix is 3.33e15."""
    if pv == "fp8":
        return 5.0e15
    return 2.0 / (1.0 / 5.0e15 + 1.0 / 2.5e15)


def fmt_ms(x: float) -> float:
    return float(f"{x:.4f}") if math.isfinite(x) else x
