"""torch.ops.telefuser_amd ops on the GPU: each gives exactly what the module-level function over the same
C-ABI entry gives (quantizers: per block with and without sm_scale or mean, per warp; attention: FP8 P.V
with per-warp / per-thread / per-block scales, smoothed V, half P.V, LSE)."""

import pytest
import torch

from tests.gpu_util import log, require_gpu
from tests.inputs import qkv

pytestmark = pytest.mark.gpu
LOG2E = 1.44269504


def test_quant_ops_match_functions():
    dev = require_gpu()
    from telefuser_amd import ops  # noqa: F401  (registers the ops)
    from telefuser_amd import sageattn2 as sa

    q, k, _ = qkv(1, 700, 515, 3, 3, seed=91, k_offset_std=0.5)
    q, k = q.to(dev), k.to(dev)
    T = torch.ops.telefuser_amd
    for lay, code in (("NHD", 0), ("HND", 1)):
        x = q if lay == "NHD" else q.transpose(1, 2).contiguous()
        kk = k if lay == "NHD" else k.transpose(1, 2).contiguous()
        b, l, h = (x.shape[0], x.shape[1], x.shape[2]) if lay == "NHD" else (x.shape[0], x.shape[2], x.shape[1])
        out = torch.empty(x.shape, dtype=torch.int8, device=dev)
        sc = torch.empty((b, h, (l + 127) // 128), dtype=torch.float32, device=dev)
        T.quant_per_block_int8_cuda_with_sm_scale(x, out, sc, 0.125 * LOG2E, 128, code)
        ro, rs = sa.quant_per_block_int8(x, 128, sm_scale=0.125 * LOG2E, tensor_layout=lay)
        assert torch.equal(out, ro) and torch.equal(sc, rs)
        T.quant_per_block_int8_cuda(x, out, sc, 128, code)
        ro, rs = sa.quant_per_block_int8(x, 128, tensor_layout=lay)
        assert torch.equal(out, ro) and torch.equal(sc, rs)
        km = sa.k_mean(kk, lay)
        ko = torch.empty(kk.shape, dtype=torch.int8, device=dev)
        ks = torch.empty((b, h, (515 + 63) // 64), dtype=torch.float32, device=dev)
        T.quant_per_block_int8_fuse_sub_mean_cuda(kk, km, ko, ks, 64, code)
        ro, rs = sa.quant_per_block_int8(kk, 64, mean=km, tensor_layout=lay)
        assert torch.equal(ko, ro) and torch.equal(ks, rs)
        ws = torch.empty((b, h, (l + 127) // 128 * 4), dtype=torch.float32, device=dev)
        T.quant_per_warp_int8_cuda(x, out, ws, 128, 32, code)
        rq, rqs, _, _ = sa.per_warp_int8(x, kk, km, tensor_layout=lay)
        assert torch.equal(out, rq) and torch.equal(ws, rqs)
    torch.cuda.synchronize()


@pytest.mark.parametrize("gran", ["per_block", "per_warp", "per_thread"])
def test_attention_ops_match_functions(gran):
    dev = require_gpu()
    from telefuser_amd import ops  # noqa: F401
    from telefuser_amd import sageattn2 as sa

    B, Lq, Lk, Hq, Hkv = 1, 900, 1300, 4, 2
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, seed=92, k_offset_std=0.5)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    sm = 128 ** -0.5
    code = {"per_block": 1, "per_warp": 2, "per_thread": 3}[gran]
    q8, qs, k8, ks, _, v8, vs, vm = sa.sage_quant(q, k, v, tensor_layout="NHD", qk_quant_gran=gran, sm_scale=sm,
                                                  smooth_v=True)
    qk_mult = 1.0 if gran == "per_block" else sm * LOG2E
    log(f"attention ops {gran}")
    T = torch.ops.telefuser_amd
    o = torch.empty(q.shape, dtype=torch.bfloat16, device=dev)
    lse = T.qk_int8_sv_f8_accum_f32_fuse_v_scale_fuse_v_mean_attn(q8, k8, v8, o, qs, ks, vs, vm, 0, 0, code, sm, 1)
    ro, rl = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, tensor_layout="NHD", out_dtype=torch.bfloat16, qk_mult=qk_mult,
                          return_lse=True, qk_quant_gran=gran, v_mean=vm)
    torch.cuda.synchronize()
    assert torch.equal(o, ro) and torch.equal(lse, rl)
    v8n, vsn, _ = sa.per_channel_fp8(v, tensor_layout="NHD", smooth_v=False)
    for name in ("qk_int8_sv_f8_accum_f32_fuse_v_scale_attn", "qk_int8_sv_f8_accum_f32_fuse_v_scale_attn_inst_buf"):
        o2 = torch.empty_like(o)
        e = getattr(T, name)(q8, k8, v8n, o2, qs, ks, vsn, 0, 0, code, sm, 0)
        r2 = sa.qattn_fwd(q8, qs, k8, ks, v8n, vsn, tensor_layout="NHD", out_dtype=torch.bfloat16, qk_mult=qk_mult,
                          qk_quant_gran=gran)
        torch.cuda.synchronize()
        assert e.numel() == 0 and torch.equal(o2, r2), name
    vt = sa.v_tile_half(v.to(torch.float16), "NHD")
    o3 = torch.empty_like(o)
    T.qk_int8_sv_f16_accum_f32_attn(q8, k8, vt, o3, qs, ks, 0, 0, code, sm, 0)
    r3 = sa.qattn_fwd(q8, qs, k8, ks, vt, None, tensor_layout="NHD", out_dtype=torch.bfloat16, qk_mult=qk_mult,
                      qk_quant_gran=gran)
    torch.cuda.synchronize()
    assert torch.equal(o3, r3)
