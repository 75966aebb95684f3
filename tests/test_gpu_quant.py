"""GPU parity of the quantizers: bit-exact against the CPU oracle (which is pinned by
tests/test_oracle_kat.py), through the C ABI."""

import numpy as np
import pytest
import torch

from tests.gpu_util import log, require_gpu, untile_v
from tests.inputs import bf16_bits, qkv

pytestmark = pytest.mark.gpu
LOG2E = 1.44269504


def _as_bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("B,Lq,Lk,Hq,Hkv,layout,dtype,variant,D", [
    (1, 1024, 1024, 2, 2, "NHD", torch.bfloat16, "cuda", 128),   # config 1
    (2, 1000, 777, 4, 2, "NHD", torch.bfloat16, "cuda", 128),    # ragged tails, GQA
    (1, 300, 130, 3, 3, "HND", torch.bfloat16, "cuda", 128),
    (1, 517, 333, 2, 1, "NHD", torch.float16, "cuda", 128),
    (1, 1000, 777, 2, 2, "NHD", torch.bfloat16, "triton", 128),
    (1, 300, 200, 2, 2, "HND", torch.float16, "triton", 128),
    (2, 1000, 777, 4, 2, "NHD", torch.bfloat16, "cuda", 64),     # head_dim 64: two rows per wave pass
    (1, 517, 333, 2, 1, "HND", torch.float16, "triton", 64),
])
def test_qk_quant_bit_exact(oracle, B, Lq, Lk, Hq, Hkv, layout, dtype, variant, D):
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    log(f"qk_quant B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} {layout} {dtype} {variant}")
    q, k, _ = qkv(B, Lq, Lk, Hq, Hkv, D=D, seed=101, k_offset_std=0.5, dtype=dtype)
    if layout == "HND":
        q, k = q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
    qd, kd = q.to(dev), k.to(dev)
    km = sa.k_mean(kd, layout)
    sm = D ** -0.5
    q8, qs, k8, ks = sa.per_block_int8(qd, kd, km, sm_scale=sm, tensor_layout=layout, variant=variant)
    torch.cuda.synchronize()
    f16 = dtype == torch.float16
    kmb = _as_bits(km)
    oq8, oqs = oracle.quant_per_block_int8(_as_bits(q), sm_scale=sm * LOG2E, blk=128, layout=layout, is_fp16=f16,
                                           variant=variant)
    ok8, oks = oracle.quant_per_block_int8(_as_bits(k), km_bits=kmb, blk=64, layout=layout, is_fp16=f16,
                                           variant=variant)
    assert np.array_equal(qs.cpu().numpy(), oqs)
    assert np.array_equal(ks.cpu().numpy(), oks)
    assert np.array_equal(q8.cpu().numpy(), oq8)
    assert np.array_equal(k8.cpu().numpy(), ok8)


@pytest.mark.parametrize("B,Lq,Lk,Hq,Hkv,layout,dtype,D", [
    (1, 1024, 1024, 2, 2, "NHD", torch.bfloat16, 128),
    (2, 1000, 777, 4, 2, "NHD", torch.bfloat16, 128),   # ragged: empty trailing warp blocks, partial key blocks
    (1, 300, 130, 3, 3, "HND", torch.bfloat16, 128),
    (1, 517, 333, 2, 1, "NHD", torch.float16, 128),
    (2, 1000, 777, 4, 2, "NHD", torch.bfloat16, 64),    # head_dim 64: a wave pass spans two warp blocks
    (1, 300, 130, 3, 3, "HND", torch.float16, 64),
])
def test_per_thread_and_per_warp_quant_bit_exact(oracle, B, Lq, Lk, Hq, Hkv, layout, dtype, D):
    """The reference's default quantizers: Triton per_thread_int8 and CUDA per_warp_int8."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    log(f"per_thread/per_warp quant B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} {layout} {dtype}")
    q, k, _ = qkv(B, Lq, Lk, Hq, Hkv, D=D, seed=102, k_offset_std=0.5, dtype=dtype)
    if layout == "HND":
        q, k = q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
    qd, kd = q.to(dev), k.to(dev)
    km = sa.k_mean(kd, layout)
    f16 = dtype == torch.float16
    kmb = _as_bits(km)
    # per thread
    q8, qs, k8, ks = sa.per_thread_int8(qd, kd, km, tensor_layout=layout)
    torch.cuda.synchronize()
    oq8, oqs = oracle.quant_per_thread_int8(_as_bits(q), layout=layout, is_fp16=f16)
    ok8, oks = oracle.quant_per_thread_int8(_as_bits(k), km_bits=kmb, is_key=True, layout=layout, is_fp16=f16)
    assert np.array_equal(qs.cpu().numpy(), oqs)
    assert np.array_equal(ks.cpu().numpy(), oks)
    assert np.array_equal(q8.cpu().numpy(), oq8)
    assert np.array_equal(k8.cpu().numpy(), ok8)
    # per warp: QuantInt8Kernel over 32-row blocks (no sm_scale), padded to 4 per 128-row block
    q8, qs, k8, ks = sa.per_warp_int8(qd, kd, km, tensor_layout=layout)
    torch.cuda.synchronize()
    oq8, oqs = oracle.quant_per_block_int8(_as_bits(q), blk=32, layout=layout, is_fp16=f16)
    ok8, oks = oracle.quant_per_block_int8(_as_bits(k), km_bits=kmb, blk=64, layout=layout, is_fp16=f16)
    n32 = oqs.shape[-1]
    qs = qs.cpu().numpy()
    assert qs.shape[-1] == (Lq + 127) // 128 * 4
    assert np.array_equal(qs[..., :n32], oqs)
    assert (qs[..., n32:] == np.float32(np.float32(1e-7) / np.float32(127.0))).all()
    assert np.array_equal(ks.cpu().numpy(), oks)
    assert np.array_equal(q8.cpu().numpy(), oq8)
    assert np.array_equal(k8.cpu().numpy(), ok8)


@pytest.mark.parametrize("B,Lq,Lk,Hq,Hkv,layout,dtype,D", [
    (1, 1024, 1024, 2, 2, "NHD", torch.bfloat16, 128),
    (2, 1000, 777, 4, 2, "NHD", torch.bfloat16, 128),   # ragged: empty trailing 16-row warps, partial K blocks
    (1, 40, 130, 3, 3, "HND", torch.bfloat16, 128),     # one 64-row Q block
    (1, 517, 333, 2, 1, "NHD", torch.float16, 128),
    (2, 1000, 777, 4, 2, "NHD", torch.bfloat16, 64),
    (1, 300, 130, 3, 3, "HND", torch.float16, 64),
])
def test_sm90_per_thread_and_per_warp_quant_bit_exact(oracle, B, Lq, Lk, Hq, Hkv, layout, dtype, D):
    """The sm90 entry's quantizer shapes (sageattn2.py:1608-1624): per_thread_int8(BLKQ=64, WARPQ=16,
    BLKK=128, WARPK=128) and per_warp_int8(BLKQ=64, WARPQ=16, BLKK=128)."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    log(f"sm90 per_thread/per_warp quant B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} {layout} {dtype}")
    q, k, _ = qkv(B, Lq, Lk, Hq, Hkv, D=D, seed=104, k_offset_std=0.5, dtype=dtype)
    if layout == "HND":
        q, k = q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
    qd, kd = q.to(dev), k.to(dev)
    km = sa.k_mean(kd, layout)
    f16 = dtype == torch.float16
    kmb = _as_bits(km)
    q8, qs, k8, ks = sa.per_thread_int8(qd, kd, km, BLKQ=64, WARPQ=16, BLKK=128, WARPK=128, tensor_layout=layout)
    torch.cuda.synchronize()
    oq8, oqs = oracle.quant_per_thread_int8(_as_bits(q), layout=layout, is_fp16=f16, sm90=True)
    ok8, oks = oracle.quant_per_thread_int8(_as_bits(k), km_bits=kmb, is_key=True, layout=layout, is_fp16=f16,
                                            sm90=True)
    assert qs.shape[-1] == (Lq + 63) // 64 * 32 and ks.shape[-1] == (Lk + 127) // 128 * 4
    assert np.array_equal(qs.cpu().numpy(), oqs)
    assert np.array_equal(ks.cpu().numpy(), oks)
    assert np.array_equal(q8.cpu().numpy(), oq8)
    assert np.array_equal(k8.cpu().numpy(), ok8)
    # per warp: QuantInt8Kernel over 16-row blocks, padded to 4 per 64-row block; K over 128-row blocks
    q8, qs, k8, ks = sa.per_warp_int8(qd, kd, km, BLKQ=64, WARPQ=16, BLKK=128, tensor_layout=layout)
    torch.cuda.synchronize()
    oq8, oqs = oracle.quant_per_block_int8(_as_bits(q), blk=16, layout=layout, is_fp16=f16)
    ok8, oks = oracle.quant_per_block_int8(_as_bits(k), km_bits=kmb, blk=128, layout=layout, is_fp16=f16)
    n16 = oqs.shape[-1]
    qs = qs.cpu().numpy()
    assert qs.shape[-1] == (Lq + 63) // 64 * 4
    assert np.array_equal(qs[..., :n16], oqs)
    assert (qs[..., n16:] == np.float32(np.float32(1e-7) / np.float32(127.0))).all()
    assert np.array_equal(ks.cpu().numpy(), oks)
    assert np.array_equal(q8.cpu().numpy(), oq8)
    assert np.array_equal(k8.cpu().numpy(), ok8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quant_nan_and_inf_inputs_match_oracle(oracle, dtype):
    """NaN elements quantize to 0 and drop out of the block maximum (cvt.rni.sat.s8 and fmaxf semantics); an
    infinite element makes its block's scale infinite and every code of the block 0."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    B, L, H = 1, 300, 2
    log(f"quant nan/inf {dtype}")
    q, k, _ = qkv(B, L, L, H, H, seed=103, k_offset_std=0.5, dtype=dtype)
    q[0, 5, 0, 7] = float("nan")     # first 32-row warp block, first 64- and 128-row block
    q[0, 70, 1, 0] = float("nan")
    q[0, 200, 0, 3] = float("inf")   # a block of its own
    k[0, 40, 1, 9] = float("nan")
    k[0, 250, 0, 1] = float("-inf")
    qd, kd = q.to(dev), k.to(dev)
    km = torch.zeros((B, H, 128), dtype=dtype, device=dev)  # a finite mean: the inf stays in one block
    f16 = dtype == torch.float16
    kmb = _as_bits(km)
    sm = 128 ** -0.5
    for variant in ("cuda", "triton"):
        q8, qs, k8, ks = sa.per_block_int8(qd, kd, km, sm_scale=sm, tensor_layout="NHD", variant=variant)
        oq8, oqs = oracle.quant_per_block_int8(_as_bits(q), sm_scale=sm * LOG2E, blk=128, layout="NHD",
                                               is_fp16=f16, variant=variant)
        ok8, oks = oracle.quant_per_block_int8(_as_bits(k), km_bits=kmb, blk=64, layout="NHD", is_fp16=f16,
                                               variant=variant)
        assert np.array_equal(q8.cpu().numpy(), oq8) and np.array_equal(k8.cpu().numpy(), ok8), variant
        assert np.array_equal(qs.cpu().numpy(), oqs) and np.array_equal(ks.cpu().numpy(), oks), variant
        assert q8.cpu()[0, 5, 0, 7].item() == 0 and k8.cpu()[0, 40, 1, 9].item() == 0
    q8, qs, k8, ks = sa.per_thread_int8(qd, kd, km, tensor_layout="NHD")
    oq8, oqs = oracle.quant_per_thread_int8(_as_bits(q), layout="NHD", is_fp16=f16)
    ok8, oks = oracle.quant_per_thread_int8(_as_bits(k), km_bits=kmb, is_key=True, layout="NHD", is_fp16=f16)
    assert np.array_equal(q8.cpu().numpy(), oq8) and np.array_equal(k8.cpu().numpy(), ok8)
    assert np.array_equal(qs.cpu().numpy(), oqs) and np.array_equal(ks.cpu().numpy(), oks)
    q8, qs, k8, ks = sa.per_warp_int8(qd, kd, km, tensor_layout="NHD")
    oq8, oqs = oracle.quant_per_block_int8(_as_bits(q), blk=32, layout="NHD", is_fp16=f16)
    assert np.array_equal(q8.cpu().numpy(), oq8)
    assert np.array_equal(qs.cpu().numpy()[..., :oqs.shape[-1]], oqs)


def test_quant_known_answers_on_gpu(oracle):
    """Closed-form cases (ties, all-zero block, tail rows) through the single-tensor entry."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    vals = torch.zeros((1, 130, 1, 128))
    vals[0, 0, 0, 0] = 127.0
    vals[0, 0, 0, 1:5] = torch.tensor([2.5, -2.5, 3.5, 0.5])
    vals[0, 64:128] = 0.0  # all-zero block
    vals[0, 128:, 0, :] = 4.0
    vals[0, 129, 0, 3] = -8.0
    x = vals.to(torch.bfloat16).to(dev)
    q8, s = sa.quant_per_block_int8(x, 64, tensor_layout="NHD")
    q8, s = q8.cpu(), s.cpu()
    assert q8[0, 0, 0, :5].tolist() == [127, 2, -2, 4, 0]
    assert s[0, 0, 1].item() == np.float32(np.float32(1e-7) / np.float32(127))
    assert q8[0, 129, 0, 3].item() == -127 and q8[0, 128, 0, 0].item() == 64
    t8, ts = sa.quant_per_block_int8(x, 64, tensor_layout="NHD", variant="triton")
    assert t8.cpu()[0, 0, 0, :5].tolist() == [127, 3, -3, 4, 1]
    assert ts.cpu()[0, 0, 1].item() == 0.0


def test_k_mean_close_to_fp64(oracle):
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    _, k, _ = qkv(2, 16, 3001, 2, 3, seed=5, k_offset_std=1.0)
    km = sa.k_mean(k.to(dev), "NHD").float().cpu().numpy()
    want = k.double().mean(dim=1).numpy()
    # bf16 result of an fp32 sum: within one bf16 ulp of the exact mean
    assert np.all(np.abs(km - want) <= np.abs(want) * 2 ** -7 + 1e-6)


@pytest.mark.parametrize("B,L,H,layout,dtype", [(1, 1024, 2, "NHD", torch.bfloat16), (2, 777, 3, "NHD", torch.bfloat16),
                                                (1, 300, 2, "HND", torch.float16), (1, 64, 1, "NHD", torch.bfloat16)])
def test_v_fp8_bit_exact(oracle, B, L, H, layout, dtype):
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    log(f"v_fp8 B={B} L={L} H={H} {layout} {dtype}")
    _, _, v = qkv(B, 8, L, H, H, seed=77, dtype=dtype)
    if layout == "HND":
        v = v.transpose(1, 2).contiguous()
    v8, vs, _ = sa.per_channel_fp8(v.to(dev), tensor_layout=layout, smooth_v=False)
    torch.cuda.synchronize()
    ov8, ovs = oracle.per_channel_fp8(_as_bits(v), layout=layout, is_fp16=dtype == torch.float16)
    assert np.array_equal(vs.cpu().numpy(), ovs)
    assert np.array_equal(untile_v(v8), ov8)


@pytest.mark.parametrize("B,L,H,layout,dtype,scale_max", [(1, 1024, 2, "NHD", torch.bfloat16, 448.0),
                                                          (2, 777, 3, "NHD", torch.bfloat16, 2.25),
                                                          (1, 300, 2, "HND", torch.float16, 448.0)])
def test_v_fp8_smooth_bit_exact(oracle, B, L, H, layout, dtype, scale_max):
    """per_channel_fp8(smooth_v=True), the sub_mean form of MeanScaleKernel: the mean [B, H, D] is within
    fp32 reduction-order noise of the float64 mean; given that mean, v_scale and the e4m3 bytes are
    bit-exact (key slots past L zero)."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    log(f"v_fp8 smooth B={B} L={L} H={H} {layout} {dtype} scale_max={scale_max}")
    _, _, v = qkv(B, 8, L, H, H, seed=78, dtype=dtype)
    v = v + 0.75  # a per-channel offset for the mean to remove
    if layout == "HND":
        v = v.transpose(1, 2).contiguous()
    v = v.to(dtype)
    v8, vs, vm = sa.per_channel_fp8(v.to(dev), tensor_layout=layout, scale_max=scale_max, smooth_v=True)
    torch.cuda.synchronize()
    gvm = vm.cpu().numpy()
    _, _, fm = oracle.per_channel_fp8(_as_bits(v), layout=layout, is_fp16=dtype == torch.float16, smooth=True)
    assert np.all(np.abs(gvm - fm) <= 1e-6 * np.maximum(1.0, np.abs(fm)))
    ov8, ovs, _ = oracle.per_channel_fp8(_as_bits(v), layout=layout, is_fp16=dtype == torch.float16, smooth=True,
                                         scale_max=scale_max, mean_in=gvm)
    assert np.array_equal(vs.cpu().numpy(), ovs)
    assert np.array_equal(untile_v(v8), ov8)


@pytest.mark.parametrize("gran,smooth_k,smooth_v,scale_max,layout,dtype,shape", [
    ("per_block", True, False, 448.0, "NHD", torch.bfloat16, (1, 1024, 1024, 2, 2)),
    ("per_block", True, True, 448.0, "NHD", torch.bfloat16, (2, 1000, 777, 4, 2)),
    ("per_block", False, False, 2.25, "HND", torch.float16, (1, 300, 130, 3, 3)),
    ("per_warp", True, False, 448.0, "NHD", torch.bfloat16, (1, 517, 333, 2, 1)),
    ("per_thread", True, False, 448.0, "HND", torch.bfloat16, (2, 700, 515, 2, 2)),
    ("per_thread", False, True, 2.25, "NHD", torch.float16, (1, 129, 65, 2, 2)),
    ("per_warp_sm90", True, False, 448.0, "NHD", torch.bfloat16, (2, 1000, 777, 4, 2)),
    ("per_thread_sm90", True, False, 448.0, "HND", torch.bfloat16, (1, 517, 333, 2, 1)),
    ("per_thread_sm90", False, False, 448.0, "NHD", torch.float16, (1, 40, 130, 3, 3)),
])
def test_sage_quant_matches_separate_calls(gran, smooth_k, smooth_v, scale_max, layout, dtype, shape):
    """The fused prologue (column passes of K and V in one launch, one finalize, V FP8, K then Q INT8 in one
    launch) must give exactly what the separate entry points give: k_mean, the per_block / per_warp /
    per_thread quantizer and per_channel_fp8, with and without K / V smoothing, both V ranges."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    B, Lq, Lk, Hq, Hkv = shape
    log(f"sage_quant {gran} smooth_k={smooth_k} smooth_v={smooth_v} scale_max={scale_max} {layout} {dtype} {shape}")
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, seed=777, k_offset_std=0.5)
    qd, kd, vd = (t.to(dev).to(dtype) for t in (q, k, v))
    if layout == "HND":
        qd, kd, vd = (t.transpose(1, 2).contiguous() for t in (qd, kd, vd))
    sm = 128 ** -0.5
    sm90 = gran.endswith("_sm90")
    gran = gran.replace("_sm90", "")
    got = sa.sage_quant(qd, kd, vd, tensor_layout=layout, qk_quant_gran=gran, sm_scale=sm, smooth_k=smooth_k,
                        scale_max=scale_max, smooth_v=smooth_v, scale_layout="sm90" if sm90 else "sm89")
    km = sa.k_mean(kd, layout) if smooth_k else None
    shapes = dict(BLKQ=64, WARPQ=16, BLKK=128) if sm90 else {}
    if gran == "per_block":
        ref_qk = sa.per_block_int8(qd, kd, km, sm_scale=sm, tensor_layout=layout)
    elif gran == "per_warp":
        ref_qk = sa.per_warp_int8(qd, kd, km, tensor_layout=layout, **shapes)
    else:
        ref_qk = sa.per_thread_int8(qd, kd, km, tensor_layout=layout, **(dict(shapes, WARPK=128) if sm90 else {}))
    v8, vs, vm = sa.per_channel_fp8(vd, tensor_layout=layout, scale_max=scale_max, smooth_v=smooth_v)
    torch.cuda.synchronize()
    for name, a, b in zip(("q_int8", "q_scale", "k_int8", "k_scale"), got[:4], ref_qk):
        assert torch.equal(a, b), f"{name} differs"
    if smooth_k:
        assert torch.equal(got[4], km)
    else:
        assert got[4] is None
    assert torch.equal(got[5].view(torch.uint8), v8.view(torch.uint8))
    assert torch.equal(got[6], vs)
    if smooth_v:
        assert torch.equal(got[7], vm)
    else:
        assert got[7] is None
