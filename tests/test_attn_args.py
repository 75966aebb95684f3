"""Argument checks of sageattn2.qattn_fwd, on the CPU: operands that do not match the launch's sizes and
scale granularity are rejected before any kernel could read outside them."""

import os

import pytest
import torch

from telefuser_amd import _lib


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libqattn.so not built")


def _ops(B=1, Lq=300, Lk=200, Hq=4, Hkv=2, gran="per_block", half=False):
    from telefuser_amd.sageattn2 import BLKK, BLKQ

    nqb, nkb = -(-Lq // BLKQ), -(-Lk // BLKK)
    q8 = torch.zeros(B, Lq, Hq, 128, dtype=torch.int8)
    k8 = torch.zeros(B, Lk, Hkv, 128, dtype=torch.int8)
    qs = torch.ones(B, Hq, nqb * {"per_block": 1, "per_warp": 4, "per_thread": 32}[gran])
    ks = torch.ones(B, Hkv, nkb * (4 if gran == "per_thread" else 1))
    if half:
        v, vs = torch.zeros(B, Hkv, 128, nkb * BLKK, dtype=torch.bfloat16), None
    else:
        v, vs = torch.zeros(B, Hkv, 128, nkb * BLKK, dtype=torch.uint8), torch.ones(B, Hkv, 128)
    return q8, qs, k8, ks, v, vs


@pytest.mark.parametrize("bad", ["q_scale_gran", "k_scale_thread", "v_short", "v_noncontig", "v_scale_shape",
                                 "half_with_scale", "q_dtype", "gran_name", "out_shape"])
def test_qattn_fwd_rejects_mismatched_operands(bad):
    from telefuser_amd import sageattn2 as sa

    gran = "per_thread" if bad == "k_scale_thread" else "per_block"
    q8, qs, k8, ks, v, vs = _ops(gran=gran)
    kw = dict(tensor_layout="NHD", qk_quant_gran=gran)
    if bad == "q_scale_gran":
        kw["qk_quant_gran"] = "per_thread"  # per-block scales handed to a per-thread launch
    elif bad == "k_scale_thread":
        ks = ks[..., :ks.shape[-1] // 4].contiguous()
    elif bad == "v_short":
        v = v[..., :64].contiguous()
    elif bad == "v_noncontig":
        v = torch.zeros(v.shape[0], v.shape[1], v.shape[3], v.shape[2], dtype=v.dtype).transpose(2, 3)
    elif bad == "v_scale_shape":
        vs = vs[:, :1].contiguous()
    elif bad == "half_with_scale":
        v = v.to(torch.bfloat16)
    elif bad == "q_dtype":
        q8 = q8.to(torch.int16)
    elif bad == "gran_name":
        kw["qk_quant_gran"] = "per_tile"
    elif bad == "out_shape":
        kw["out"] = torch.empty(1, 10, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        sa.qattn_fwd(q8, qs, k8, ks, v, vs, **kw)


@pytest.mark.parametrize("bad", ["q_scale_gran", "k_scale_short", "v_scale_shape", "out_small", "v_mean_shape",
                                 "out_dtype"])
def test_ops_reject_mismatched_operands(bad):
    """torch.ops.telefuser_amd attention ops run the same operand checks as qattn_fwd before any launch."""
    from telefuser_amd import ops  # noqa: F401  (registers the ops)

    q8, qs, k8, ks, v, vs = _ops()
    out = torch.empty(q8.shape, dtype=torch.bfloat16)
    gran, vm = 1, None
    if bad == "q_scale_gran":
        gran = 3  # per-block scales handed to a per-thread launch
    elif bad == "k_scale_short":
        ks = ks[..., :1].contiguous()
    elif bad == "v_scale_shape":
        vs = vs[:, :1].contiguous()
    elif bad == "out_small":
        out = torch.empty(1, 10, 4, 128, dtype=torch.bfloat16)
    elif bad == "v_mean_shape":
        vm = torch.zeros(1, 1, 128)
    elif bad == "out_dtype":
        out = torch.empty(q8.shape, dtype=torch.float32)
    with pytest.raises(ValueError):
        if vm is None:
            torch.ops.telefuser_amd.qk_int8_sv_f8_accum_f32_fuse_v_scale_attn(q8, k8, v, out, qs, ks, vs, 0, 0, gran,
                                                                             128 ** -0.5, 0)
        else:
            torch.ops.telefuser_amd.qk_int8_sv_f8_accum_f32_fuse_v_scale_fuse_v_mean_attn(
                q8, k8, v, out, qs, ks, vs, vm, 0, 0, gran, 128 ** -0.5, 0)


@pytest.mark.parametrize("bad", ["input_dtype", "mean_size", "scale_shape"])
def test_quant_ops_reject_bad_arguments(bad):
    from telefuser_amd import ops  # noqa: F401

    x = torch.zeros(1, 200, 2, 128, dtype=torch.bfloat16)
    out = torch.empty(x.shape, dtype=torch.int8)
    scale = torch.empty(1, 2, 4, dtype=torch.float32)
    mean = torch.zeros(1, 2, 128, dtype=torch.bfloat16)
    if bad == "input_dtype":
        x = x.float()
    elif bad == "mean_size":
        mean = torch.zeros(1, 3, 128, dtype=torch.bfloat16)
    elif bad == "scale_shape":
        scale = torch.empty(1, 2, 3, dtype=torch.float32)
    with pytest.raises(ValueError):
        torch.ops.telefuser_amd.quant_per_block_int8_fuse_sub_mean_cuda(x, mean, out, scale, 64, 0)


@pytest.mark.parametrize("bad", ["sm89_tables", "per_block", "layout_name"])
def test_qattn_fwd_sm90_layout_checks(bad):
    """scale_layout="sm90" takes per-warp / per-thread tables of the sm90 block shapes only."""
    from telefuser_amd import sageattn2 as sa

    q8, qs, k8, ks, v, vs = _ops(Lq=300, Lk=200, gran="per_thread")  # sm89 shapes: 3*32 / 4*4 entries
    kw = dict(tensor_layout="NHD", qk_quant_gran="per_thread", scale_layout="sm90")
    if bad == "per_block":
        q8, qs, k8, ks, v, vs = _ops(gran="per_block")
        kw["qk_quant_gran"] = "per_block"
    elif bad == "layout_name":
        kw["scale_layout"] = "sm100"
    with pytest.raises(ValueError):
        sa.qattn_fwd(q8, qs, k8, ks, v, vs, **kw)


@pytest.mark.parametrize("bad", ["small_grid_long_keys", "int8_q", "k_scale_gran", "no_v_scale"])
def test_fwd_q16_rejects(bad):
    """qattn_fwd_q16 takes half Q, K scales of its granularity and the e4m3 V tile, for launches the resident
    or ping-pong kernel runs (300 queries of 4 heads over 600 keys run the one-block kernel)."""
    from telefuser_amd import sageattn2 as sa

    lk = 600 if bad == "small_grid_long_keys" else 300
    q8, qs, k8, ks, v, vs = _ops(Lk=lk, gran="per_thread")
    q = torch.zeros(q8.shape, dtype=torch.bfloat16)
    kw = dict(tensor_layout="NHD", qk_quant_gran="per_thread")
    if bad == "int8_q":
        q = q8
    elif bad == "k_scale_gran":
        ks = ks[..., : ks.shape[-1] // 4].contiguous()
    elif bad == "no_v_scale":
        vs = None
    with pytest.raises(ValueError):
        sa.qattn_fwd_q16(q, k8, ks, v, vs, **kw)


def test_q16_supported_rule():
    """The host rule behind the drop-in's route: every granularity on the resident kernel (at most 512 keys)
    and on the ping-pong kernel, nothing on the one-block kernel; head_dim 128, or 64 (always the ping-pong
    kernel)."""
    from telefuser_amd import sageattn2 as sa

    for gran in ("per_block", "per_warp", "per_thread"):
        assert sa.q16_supported(1, 1000, 512, 4, 128, gran, False)  # resident
        assert sa.q16_supported(1, 32760, 32760, 12, 128, gran, False)  # ping-pong (C2)
        assert not sa.q16_supported(1, 300, 600, 4, 128, gran, False)  # one-block
        assert sa.q16_supported(1, 1000, 512, 4, 64, gran, False)  # head_dim 64: the ping-pong kernel's form
        assert not sa.q16_supported(1, 1000, 512, 4, 96, gran, False)
