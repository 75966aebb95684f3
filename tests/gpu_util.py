"""Helpers shared by the GPU parity tests."""

import numpy as np
import pytest
import torch


def vtile_pos(kappa):
    """Storage position of key kappa inside a 64-key tile of the FP8 V layout (include/qattn.h)."""
    kappa = np.asarray(kappa)
    kb, g, hf, t = kappa >> 5, (kappa >> 3) & 3, (kappa >> 2) & 1, kappa & 3
    return hf * 32 + kb * 16 + g * 4 + t


POS = vtile_pos(np.arange(64))


def untile_v(v8_dev: torch.Tensor) -> np.ndarray:
    """[B, H, D, Lpad] tile-permuted e4m3 bytes -> the same in plain key order."""
    a = v8_dev.view(torch.uint8).cpu().numpy()
    B, H, D, Lp = a.shape
    t = a.reshape(B, H, D, Lp // 64, 64)
    return np.ascontiguousarray(t[..., POS].reshape(B, H, D, Lp))


def require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from telefuser_amd import _lib

    _lib.load()  # raises if the HIP library was not built: never silently fall back
    return "cuda:0"


def log(msg):
    print(msg, flush=True)
