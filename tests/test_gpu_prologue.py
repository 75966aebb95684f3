"""Fused RMSNorm + RoPE + INT8 prologue on the GPU: bit-exact against the oracle (norm_rope, then the
per-block quantizer), and the fused Wan self-attention against the unfused path."""

import numpy as np
import pytest
import torch

from tests.gpu_util import log, require_gpu
from tests.inputs import bf16_bits, cosine

pytestmark = pytest.mark.gpu
LOG2E = 1.44269504


def _inputs(B, L, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    xq = (torch.randn((B, L, H * D), generator=g) * 2).to(torch.bfloat16)
    xk = (torch.randn((B, L, H * D), generator=g) * 2 + 0.3).to(torch.bfloat16)
    xv = torch.randn((B, L, H * D), generator=g).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn((H * D,), generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn((H * D,), generator=g)).to(torch.bfloat16)
    ang = torch.rand((L, 1, D // 2), generator=g, dtype=torch.float64) * 6.3  # the reference's fp64 freqs
    return xq, xk, xv, wq, wk, ang.cos(), ang.sin()


@pytest.mark.parametrize("B,L,H", [(1, 300, 2), (2, 777, 3)])
def test_prologue_bit_exact(oracle, B, L, H):
    dev = require_gpu()
    from telefuser_amd.prologue import norm_rope_quant_qk

    D = 128
    xq, xk, xv, wq, wk, fc, fs = _inputs(B, L, H, D, seed=L)
    log(f"prologue B={B} L={L} H={H}")
    q8, qs, k8, ks, km = norm_rope_quant_qk(*(t.to(dev) for t in (xq, xk, wq, wk, fc, fs)), num_heads=H)
    torch.cuda.synchronize()
    cs, sn = fc.reshape(L, -1).float().numpy(), fs.reshape(L, -1).float().numpy()
    qn = oracle.norm_rope(bf16_bits(xq), bf16_bits(wq), cs, sn, D).reshape(B, L, H, D)
    kn = oracle.norm_rope(bf16_bits(xk), bf16_bits(wk), cs, sn, D).reshape(B, L, H, D)
    kmb = km.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    # the smoothing vector: the mean of the rotated K, to one bf16 rounding of the fp64 mean
    km_ref = oracle.bf16_bits_to_f32(oracle.k_mean_bits(kn))
    assert np.abs(oracle.bf16_bits_to_f32(kmb) - km_ref).max() <= np.abs(km_ref).max() * 2 ** -8
    oq8, oqs = oracle.quant_per_block_int8(qn, sm_scale=D ** -0.5 * LOG2E, blk=128)
    ok8, oks = oracle.quant_per_block_int8(kn, km_bits=kmb, blk=64)
    assert np.array_equal(qs.cpu().numpy(), oqs) and np.array_equal(q8.cpu().numpy(), oq8)
    assert np.array_equal(ks.cpu().numpy(), oks) and np.array_equal(k8.cpu().numpy(), ok8)


def test_fused_wan_self_attention_matches_unfused(oracle):
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa
    from telefuser_amd.prologue import wan_self_attention

    B, L, H, D = 1, 1000, 2, 128
    xq, xk, xv, wq, wk, fc, fs = _inputs(B, L, H, D, seed=5)
    o = wan_self_attention(*(t.to(dev) for t in (xq, xk, xv, wq, wk, fc, fs)), num_heads=H)
    # the unfused route: norm and rope materialised (oracle), then the drop-in sage call
    cs, sn = fc.reshape(L, -1).float().numpy(), fs.reshape(L, -1).float().numpy()
    to_t = lambda bits: torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).reshape(B, L, H, D)
    qn = to_t(oracle.norm_rope(bf16_bits(xq), bf16_bits(wq), cs, sn, D))
    kn = to_t(oracle.norm_rope(bf16_bits(xk), bf16_bits(wk), cs, sn, D))
    vn = xv.reshape(B, L, H, D)
    o2 = sa.sageattn_qk_int8_pv_fp8_cuda(qn.to(dev), kn.to(dev), vn.to(dev), tensor_layout="NHD",
                                         qk_quant_gran="per_block", pv_accum_dtype="fp32+fp32")
    torch.cuda.synchronize()
    truth = oracle.attn_fp64(bf16_bits(qn), bf16_bits(kn), bf16_bits(vn), D ** -0.5)
    a, b = o.float().cpu().numpy().reshape(B, L, H, D), o2.float().cpu().numpy()
    log(f"fused vs unfused cos={cosine(a, b):.7f} fused vs truth cos={cosine(a, truth):.6f}")
    assert cosine(a, b) >= 0.99999
    assert cosine(a, truth) >= 0.999
