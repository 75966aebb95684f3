"""The op-level schemas of tf-kernel's SageAttention extension (tf-kernel/csrc/common_extension.cc:168-260),
registered as ``torch.ops.telefuser_amd.<name>`` over the C ABI of libqattn, so code and tests that call the
reference at op granularity (``torch.ops.tf_kernel.<name>``) can switch namespaces.

Same names, argument order and meaning, in-place outputs (``Tensor!``) and returned LSE (log2 domain,
[B, Hq, Lq], an empty tensor when return_lse is 0).  Deliberate differences:
  * ``value`` of the attention ops is V in this library's tile layout: e4m3 [B, Hkv, D, Lpad] from
    ``per_channel_fp8`` / ``qattn_sage_quant`` for the f8 ops, or the half tile from ``v_tile_half`` for the
    f16 ops (the reference's ops take the NVIDIA mma permutation of ``transpose_pad_permute_cuda``).
  * ``qk_quant_gran`` takes the reference's codes 2 (per warp) and 3 (per thread), for which the kernel
    applies ``sm_scale``·log2(e), and also 1 (per block: sm_scale·log2(e) already folded into Q).
  * every ``*_accum_f16*`` / ``*_inst_buf`` variant accumulates P.V in fp32 (MFMA accumulators are fp32).
  * ``quant_per_warp_int8_cuda`` supports the reference's shape block_size = 128, warp_block_size = 32.
The ops launch on the current stream and never synchronise; the library is loaded on first use.
"""

from __future__ import annotations

import torch

from . import _lib
from . import sageattn2 as _sa

LOG2E = 1.44269504
_LAYOUT = {0: "NHD", 1: "HND"}


def _layout(code: int) -> str:
    if code not in _LAYOUT:
        raise ValueError(f"tensor_layout must be 0 (NHD) or 1 (HND), got {code}")
    return _LAYOUT[code]


def _dims(x: torch.Tensor, layout: str):
    if layout == "NHD":
        b, l, h, d = x.shape
    else:
        b, h, l, d = x.shape
    return b, l, h, d


def _check_input(inp):
    if inp.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"input must be bfloat16 or float16, got {inp.dtype}")
    if inp.dim() != 4 or inp.stride(-1) != 1:
        raise ValueError("input must be a 4-D tensor with a contiguous last dimension")


def _quant(inp, mean, out, scale, sm_scale, has_sm, block_size, tensor_layout):
    L = _lib.load()
    lay = _layout(tensor_layout)
    _check_input(inp)
    b, l, h, d = _dims(inp, lay)
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    if scale.shape != (b, h, (l + block_size - 1) // block_size) or scale.dtype != torch.float32:
        raise ValueError("scale must be float32 [B, H, ceil(L / block_size)]")
    if out.shape != inp.shape or out.dtype != torch.int8:
        raise ValueError("output must be int8 with the input's shape")
    mc = None
    if mean is not None:
        if mean.numel() != b * h * d or not mean.is_floating_point() or mean.device != inp.device:
            raise ValueError(f"mean must be a floating-point [B, H, D] = {(b, h, d)} tensor (or a keepdim form) on "
                             f"{inp.device}, got {mean.dtype} {tuple(mean.shape)} on {mean.device}")
        mc = mean.to(inp.dtype).reshape(b, h, d).contiguous()
    _lib.check(L.qattn_quant_per_block_int8(
        _lib.seq(inp, lay), _lib.dtype_code(inp.dtype), b, l, h, d, _lib.ptr(mc), _lib.seq(out, lay), _lib.ptr(scale),
        float(sm_scale), int(has_sm), int(block_size), _lib.QATTN_QUANT_CUDA, _lib.stream_of(inp)))


@torch.library.custom_op("telefuser_amd::quant_per_block_int8_cuda_with_sm_scale", mutates_args=("output", "scale"))
def quant_per_block_int8_cuda_with_sm_scale(input: torch.Tensor, output: torch.Tensor, scale: torch.Tensor,
                                            sm_scale: float, block_size: int, tensor_layout: int) -> None:
    """QuantInt8Kernel with the input multiplied by sm_scale (fused.cu:59-194)."""
    _quant(input, None, output, scale, sm_scale, 1, block_size, tensor_layout)


@torch.library.custom_op("telefuser_amd::quant_per_block_int8_cuda", mutates_args=("output", "scale"))
def quant_per_block_int8_cuda(input: torch.Tensor, output: torch.Tensor, scale: torch.Tensor, block_size: int,
                              tensor_layout: int) -> None:
    """QuantInt8Kernel without a scale factor."""
    _quant(input, None, output, scale, 0.0, 0, block_size, tensor_layout)


@torch.library.custom_op("telefuser_amd::quant_per_block_int8_fuse_sub_mean_cuda", mutates_args=("output", "scale"))
def quant_per_block_int8_fuse_sub_mean_cuda(input: torch.Tensor, mean: torch.Tensor, output: torch.Tensor,
                                            scale: torch.Tensor, block_size: int, tensor_layout: int) -> None:
    """QuantInt8Kernel of input - mean (mean [B, H, D] or a keepdim form, in the input's dtype)."""
    _quant(input, mean, output, scale, 0.0, 0, block_size, tensor_layout)


@torch.library.custom_op("telefuser_amd::quant_per_warp_int8_cuda", mutates_args=("output", "scale"))
def quant_per_warp_int8_cuda(input: torch.Tensor, output: torch.Tensor, scale: torch.Tensor, block_size: int,
                             warp_block_size: int, tensor_layout: int) -> None:
    """Per-warp Q quantization (quant_per_warp_int8_cuda): one scale per 32-row warp block of every 128-row
    block, scale [B, H, ceil(L / 128) * 4]."""
    if block_size != 128 or warp_block_size != 32:
        raise ValueError("quant_per_warp_int8_cuda supports block_size 128 with warp_block_size 32")
    L = _lib.load()
    lay = _layout(tensor_layout)
    _check_input(input)
    b, l, h, d = _dims(input, lay)
    if scale.shape != (b, h, (l + 127) // 128 * 4) or scale.dtype != torch.float32:
        raise ValueError("scale must be float32 [B, H, ceil(L / 128) * 4]")
    if output.shape != input.shape or output.dtype != torch.int8:
        raise ValueError("output must be int8 with the input's shape")
    empty = torch.empty((b, 0, h, d) if lay == "NHD" else (b, h, 0, d), dtype=input.dtype, device=input.device)
    empty8 = torch.empty(empty.shape, dtype=torch.int8, device=input.device)
    dummy = torch.empty(1, dtype=torch.float32, device=input.device)
    _lib.check(L.qattn_quant_qk_per_warp_int8(
        _lib.seq(input, lay), _lib.seq(empty, lay), _lib.dtype_code(input.dtype), b, l, 0, h, h, d, None,
        _lib.seq(output, lay), _lib.seq(empty8, lay), _lib.ptr(scale), _lib.ptr(dummy), _lib.stream_of(input)))


def _attn(query, key, value, output, query_scale, key_scale, value_scale, value_mean, tensor_layout, is_causal,
          qk_quant_gran, sm_scale, return_lse):
    L = _lib.load()
    lay = _layout(tensor_layout)
    if qk_quant_gran not in (1, 2, 3):
        raise ValueError(f"qk_quant_gran must be 1 (per block), 2 (per warp) or 3 (per thread), got {qk_quant_gran}")
    b, lq, hq, d = _dims(query, lay)
    _, lk, hkv, _ = _dims(key, lay)
    if value_scale is not None:
        v_kind = _lib.QATTN_V_FP8
    else:
        v_kind = _lib.QATTN_V_BF16 if value.dtype == torch.bfloat16 else _lib.QATTN_V_FP16
    lpad = value.shape[-1]
    if value.dim() != 4:
        raise ValueError(f"value must be this library's V tile layout [B, Hkv, D, Lpad] = {(b, hkv, d)} + Lpad")
    # the same checks as the module's qattn_fwd (scale shapes per granularity, V tile, output), so that no
    # operand of another granularity or size reaches the kernel (the reference's CHECK_SHAPE / CHECK_DTYPE,
    # sm89_qk_int8_sv_f8_accum_f32_attn_inst_buf.cu:125-129)
    gran = {1: "per_block", 2: "per_warp", 3: "per_thread"}[qk_quant_gran]
    if not output.is_floating_point() or output.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"output must be bfloat16 or float16, got {output.dtype}")
    _sa._check_attn_operands(query, query_scale, key, key_scale, value, value_scale, b, lq, lk, hq, hkv, d, gran,
                             output, output.dtype)
    if value_mean is not None and (value_scale is None or value_mean.dtype != torch.float32 or
                                   tuple(value_mean.shape) != (b, hkv, d) or not value_mean.is_contiguous() or
                                   value_mean.device != query.device):
        raise ValueError(f"value_mean must be a contiguous float32 tensor of shape {(b, hkv, d)} (FP8 V only)")
    qk_mult = 1.0 if qk_quant_gran == 1 else float(sm_scale) * LOG2E
    lse = torch.empty((b, hq, lq) if return_lse else (0,), dtype=torch.float32, device=query.device)
    ns = L.qattn_fwd_ex_num_splits(b, lq, lk, hq, v_kind, qk_quant_gran)
    wsb = L.qattn_fwd_workspace_size(b, lq, hq, d, ns)
    ws = torch.empty(wsb, dtype=torch.uint8, device=query.device) if wsb else None
    _lib.check(L.qattn_fwd_ex2(
        _lib.seq(query, lay), _lib.ptr(query_scale), _lib.seq(key, lay), _lib.ptr(key_scale), _lib.ptr(value), v_kind,
        lpad, _lib.ptr(value_scale), _lib.ptr(value_mean), _lib.seq(output, lay), _lib.dtype_code(output.dtype), b,
        lq, lk, hq, hkv, d, qk_mult, int(qk_quant_gran), int(is_causal), 0, None,
        _lib.ptr(lse) if return_lse else None, ns, _lib.ptr(ws), wsb, _lib.stream_of(query)))
    return lse


def _def_f8(name: str, doc: str):
    @torch.library.custom_op(f"telefuser_amd::{name}", mutates_args=("output",))
    def op(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, output: torch.Tensor,
           query_scale: torch.Tensor, key_scale: torch.Tensor, value_scale: torch.Tensor, tensor_layout: int,
           is_causal: int, qk_quant_gran: int, sm_scale: float, return_lse: int) -> torch.Tensor:
        return _attn(query, key, value, output, query_scale, key_scale, value_scale, None, tensor_layout, is_causal,
                     qk_quant_gran, sm_scale, return_lse)
    op.__doc__ = doc
    return op


def _def_f8_mean(name: str, doc: str):
    @torch.library.custom_op(f"telefuser_amd::{name}", mutates_args=("output",))
    def op(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, output: torch.Tensor,
           query_scale: torch.Tensor, key_scale: torch.Tensor, value_scale: torch.Tensor, value_mean: torch.Tensor,
           tensor_layout: int, is_causal: int, qk_quant_gran: int, sm_scale: float, return_lse: int) -> torch.Tensor:
        return _attn(query, key, value, output, query_scale, key_scale, value_scale, value_mean, tensor_layout,
                     is_causal, qk_quant_gran, sm_scale, return_lse)
    op.__doc__ = doc
    return op


def _def_f16(name: str, doc: str):
    @torch.library.custom_op(f"telefuser_amd::{name}", mutates_args=("output",))
    def op(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, output: torch.Tensor,
           query_scale: torch.Tensor, key_scale: torch.Tensor, tensor_layout: int, is_causal: int,
           qk_quant_gran: int, sm_scale: float, return_lse: int) -> torch.Tensor:
        return _attn(query, key, value, output, query_scale, key_scale, None, None, tensor_layout, is_causal,
                     qk_quant_gran, sm_scale, return_lse)
    op.__doc__ = doc
    return op


# FP8 P.V (sm89 kernels, qk_int_sv_f8_cuda_sm89.cuh; common_extension.cc:239-258 and the inst_buf forms)
qk_int8_sv_f8_accum_f32_fuse_v_scale_attn = _def_f8(
    "qk_int8_sv_f8_accum_f32_fuse_v_scale_attn", "INT8 Q.K^T, FP8 P.V, v_scale epilogue.")
qk_int8_sv_f8_accum_f32_fuse_v_scale_attn_inst_buf = _def_f8(
    "qk_int8_sv_f8_accum_f32_fuse_v_scale_attn_inst_buf", "As qk_int8_sv_f8_accum_f32_fuse_v_scale_attn.")
qk_int8_sv_f8_accum_f16_fuse_v_scale_attn_inst_buf = _def_f8(
    "qk_int8_sv_f8_accum_f16_fuse_v_scale_attn_inst_buf",
    "As qk_int8_sv_f8_accum_f32_fuse_v_scale_attn (P.V accumulated in fp32; quantize V with scale_max 2.25 "
    "as the reference's fp32+fp16 path does).")
qk_int8_sv_f8_accum_f32_fuse_v_scale_fuse_v_mean_attn = _def_f8_mean(
    "qk_int8_sv_f8_accum_f32_fuse_v_scale_fuse_v_mean_attn", "FP8 P.V of smoothed V, v_mean added back.")
# half P.V (sm80 kernels; common_extension.cc:196-231): value is the half tile of v_tile_half
qk_int8_sv_f16_accum_f32_attn = _def_f16("qk_int8_sv_f16_accum_f32_attn", "INT8 Q.K^T, half P.V in fp32.")
qk_int8_sv_f16_accum_f16_attn = _def_f16(
    "qk_int8_sv_f16_accum_f16_attn", "As qk_int8_sv_f16_accum_f32_attn (fp32 accumulation).")
qk_int8_sv_f16_accum_f16_attn_inst_buf = _def_f16(
    "qk_int8_sv_f16_accum_f16_attn_inst_buf", "As qk_int8_sv_f16_accum_f32_attn (fp32 accumulation).")

OPS = (
    "quant_per_block_int8_cuda_with_sm_scale",
    "quant_per_block_int8_cuda",
    "quant_per_block_int8_fuse_sub_mean_cuda",
    "quant_per_warp_int8_cuda",
    "qk_int8_sv_f8_accum_f32_fuse_v_scale_attn",
    "qk_int8_sv_f8_accum_f32_fuse_v_scale_attn_inst_buf",
    "qk_int8_sv_f8_accum_f16_fuse_v_scale_attn_inst_buf",
    "qk_int8_sv_f8_accum_f32_fuse_v_scale_fuse_v_mean_attn",
    "qk_int8_sv_f16_accum_f32_attn",
    "qk_int8_sv_f16_accum_f16_attn",
    "qk_int8_sv_f16_accum_f16_attn_inst_buf",
)
