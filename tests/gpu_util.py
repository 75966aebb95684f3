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


def lse_max_err(lse, ref_lse, out=None) -> float:
    """Max |lse - ref_lse| over the rows that have keys, after checking the rows that have none.

    A row with no valid key has LSE -inf on both sides (log of an empty sum) and, when `out` is given
    ([..., rows, D] aligned with the LSE's rows), an all-zero output row.  No NaN is accepted on either
    side, so a kernel that wrote NaN or a finite value for an empty row fails here."""
    lse = np.asarray(lse, np.float64)
    ref_lse = np.asarray(ref_lse, np.float64)
    assert lse.shape == ref_lse.shape, (lse.shape, ref_lse.shape)
    assert not np.isnan(lse).any(), "NaN in the kernel's LSE"
    assert not np.isnan(ref_lse).any(), "NaN in the oracle's LSE"
    empty = np.isneginf(ref_lse)
    assert np.array_equal(np.isneginf(lse), empty), "rows without keys differ between kernel and oracle"
    assert not np.isposinf(lse).any()
    if out is not None and empty.any():
        o = np.asarray(out)
        assert np.all(o[empty] == 0), "a row without keys has a non-zero output"
    fin = ~empty
    return float(np.abs(lse[fin] - ref_lse[fin]).max()) if fin.any() else 0.0
