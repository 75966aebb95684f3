"""Fused prologue of the Wan self-attention: RMSNorm + 3-D RoPE + INT8 quantization of Q and K.

The reference runs ``q = rope_apply(norm_q(self.q(x)))`` (and the same for K) as separate kernels and
then quantizes inside the attention call (telefuser/models/wan_video_dit.py:196-207, norm_infer in
telefuser/kernel/triton/norm.py:469-507, the interleaved rotary kernel in
telefuser/kernel/triton/rotary.py:21-88).  Here the linear outputs go straight to INT8: a per-row
RMSNorm statistic pass, one pass for the K mean of the rotated values, and one quantizer launch that
applies norm + RoPE to every chunk it loads, so the normalized / rotated bf16 tensors never reach HBM.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from . import sageattn2 as sa


def _cos_sin(freqs_cos: torch.Tensor, freqs_sin: torch.Tensor, L: int, half: int, device):
    cs = freqs_cos.reshape(L, half).to(device=device, dtype=torch.float32).contiguous()
    sn = freqs_sin.reshape(L, half).to(device=device, dtype=torch.float32).contiguous()
    return cs, sn


def row_rstd(x: torch.Tensor, eps: float) -> torch.Tensor:
    """1 / sqrt(mean(x^2, -1) + eps) per row of x [..., N] (fp32, shape x.shape[:-1])."""
    L = _lib.load()
    n = x.shape[-1]
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    out = torch.empty(x2.shape[0], dtype=torch.float32, device=x.device)
    _lib.check(L.qattn_row_rstd(_lib.ptr(x2), _lib.dtype_code(x.dtype), x2.shape[0], x2.stride(0), n, float(eps),
                                _lib.ptr(out), _lib.stream_of(x)))
    return out.reshape(x.shape[:-1])


def norm_rope_quant_qk(xq: torch.Tensor, xk: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor,
                       freqs_cos: torch.Tensor, freqs_sin: torch.Tensor, num_heads: int, eps: float = 1e-6,
                       sm_scale: Optional[float] = None, smooth_k: bool = True, variant: str = "cuda"):
    """xq, xk: linear outputs [B, L, H*D]; wq, wk: RMSNorm weights [H*D]; freqs_cos / freqs_sin: [L, 1, D/2]
    (or [L, D/2]).  Returns (q_int8 [B, L, H, D], q_scale [B, H, ceil(L/128)], k_int8, k_scale
    [B, H, ceil(L/64)], km [B, H, D] or None) - the operands ``qattn_fwd`` takes (NHD), i.e. what
    ``per_block_int8`` would produce from the normalized, rotated Q and K."""
    L = _lib.load()
    if xq.shape != xk.shape or xq.dim() != 3 or xq.dtype != xk.dtype:
        raise ValueError("xq and xk must both be [B, L, H*D] of one dtype")
    b, l, n = xq.shape
    h = num_heads
    d = n // h
    if d * h != n or d not in (64, 128):
        raise ValueError(f"H*D = {n} with {h} heads gives head_dim {d}; 64 or 128 supported")
    xq4, xk4 = xq.reshape(b, l, h, d), xk.reshape(b, l, h, d)
    cs, sn = _cos_sin(freqs_cos, freqs_sin, l, d // 2, xq.device)
    wq, wk = wq.to(xq.dtype).contiguous(), wk.to(xq.dtype).contiguous()
    rq, rk = row_rstd(xq, eps), row_rstd(xk, eps)
    dt = _lib.dtype_code(xq.dtype)
    km = None
    if smooth_k:
        km = torch.empty((b, h, d), dtype=xq.dtype, device=xq.device)
        ws = torch.empty(L.qattn_seq_mean_workspace_size(b, l, h, d), dtype=torch.uint8, device=xq.device)
        _lib.check(L.qattn_norm_rope_seq_mean(_lib.seq(xk4, "NHD"), dt, b, l, h, d, _lib.ptr(rk), _lib.ptr(wk),
                                              _lib.ptr(cs), _lib.ptr(sn), cs.stride(0), _lib.ptr(km), _lib.ptr(ws),
                                              ws.numel(), _lib.stream_of(xq)))
    q8 = torch.empty((b, l, h, d), dtype=torch.int8, device=xq.device)
    k8 = torch.empty_like(q8)
    q_scale = torch.empty((b, h, (l + sa.BLKQ - 1) // sa.BLKQ), dtype=torch.float32, device=xq.device)
    k_scale = torch.empty((b, h, (l + sa.BLKK - 1) // sa.BLKK), dtype=torch.float32, device=xq.device)
    if sm_scale is None:
        sm_scale = d ** -0.5
    var = _lib.QATTN_QUANT_TRITON if variant == "triton" else _lib.QATTN_QUANT_CUDA
    _lib.check(L.qattn_norm_rope_quant_qk(
        _lib.seq(xq4, "NHD"), _lib.seq(xk4, "NHD"), dt, b, l, h, d, _lib.ptr(rq), _lib.ptr(rk), _lib.ptr(wq),
        _lib.ptr(wk), _lib.ptr(cs), _lib.ptr(sn), cs.stride(0), _lib.ptr(km), _lib.seq(q8, "NHD"),
        _lib.seq(k8, "NHD"), _lib.ptr(q_scale), _lib.ptr(k_scale), float(sm_scale * sa.LOG2E), var,
        _lib.stream_of(xq)))
    return q8, q_scale, k8, k_scale, km


def wan_self_attention(xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor,
                       freqs_cos: torch.Tensor, freqs_sin: torch.Tensor, num_heads: int, eps: float = 1e-6,
                       kv_valid_len=None) -> torch.Tensor:
    """Wan self-attention from the three linear outputs [B, L, H*D] to the attention output [B, L, H*D]
    (the lines between the projections and ``self.o`` in wan_video_dit.py:196-215), with the fused
    prologue, per-channel FP8 V and the INT8-QK / FP8-PV kernel."""
    b, l, n = xq.shape
    d = n // num_heads
    q8, qs, k8, ks, _ = norm_rope_quant_qk(xq, xk, wq, wk, freqs_cos, freqs_sin, num_heads, eps)
    v8, vs, _ = sa.per_channel_fp8(xv.reshape(b, l, num_heads, d), tensor_layout="NHD", smooth_v=False)
    o = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, tensor_layout="NHD", out_dtype=xq.dtype, kv_valid_len=kv_valid_len)
    return o.reshape(b, l, n)


__all__ = ["row_rstd", "norm_rope_quant_qk", "wan_self_attention"]
