"""SageAttention-2 compatible front end over the gfx950 kernels of libqattn.

Mirrors the module TeleFuser's backend registry loads into ``backends.sageattention``
(telefuser/ops/attention/backends.py:87-99, called from attention_impl.py:245-283), i.e. the public
functions of tf-kernel/tf_kernel/sageattn2.py: ``per_block_int8`` (:96-187), ``per_channel_fp8``
(:320-407), ``sageattn_qk_int8_pv_fp8_cuda`` (:1197-1457), ``sageattn_qk_int8_pv_fp8_cuda_sm90``
(:1460-1693), ``sageattn_qk_int8_pv_fp16_cuda`` (:930-1194), ``sageattn_varlen`` (:772-927) and
``sageattn`` (:415-548).

Differences from the reference, all deliberate:
  * ``qk_quant_gran`` selects the reference's quantizer: "per_thread" (the default, Triton
    quant_per_thread.py), "per_warp" (CUDA quant_per_warp_int8) or the extra "per_block" (CUDA
    QuantInt8Kernel with sm_scale*log2e folded into Q).  Per-warp Q blocks are always 32 rows (the
    reference uses 16 for head_dim 128 with "fp16+fp32" accumulation).
  * ``pv_accum_dtype`` variants all accumulate P.V in full fp32 (MFMA accumulators are fp32); they keep
    the reference's other semantics: "fp32" honours ``smooth_v``, "fp32+fp32" and "fp32+fp16" ignore it
    with the reference's warning, and "fp32+fp16" quantizes V with scale_max 2.25 (448 otherwise).
  * ``kv_valid_len`` (per-batch number of valid keys) is honoured; ``attn_mask`` is ignored exactly as
    the reference CUDA functions ignore it (it is swallowed by ``**kwargs``).
  * ``per_channel_fp8`` returns V in this library's tile layout [B, H, D, Lpad] for both tensor
    layouts (see include/qattn.h), not the NVIDIA mma permutation.
"""

from __future__ import annotations

import warnings
from typing import Any, Optional

import torch

from . import _lib

LOG2E = 1.44269504  # the constant the reference folds into sm_scale (sageattn2.py:177)
BLKQ = 128
BLKK = 64


def _dims(x: torch.Tensor, layout: str):
    if layout == "NHD":
        b, l, h, d = x.shape
    elif layout == "HND":
        b, h, l, d = x.shape
    else:
        raise ValueError(f"Unknown tensor layout: {layout}")
    return b, l, h, d


def _mean_3d(km: torch.Tensor, b: int, h: int, d: int, layout: str) -> torch.Tensor:
    """Accept km as [B, H, D] or the keepdim forms [B, 1, H, D] (NHD) / [B, H, 1, D] (HND)."""
    if km.dim() == 4:
        km = km.squeeze(1) if layout == "NHD" else km.squeeze(2)
    if tuple(km.shape) != (b, h, d):
        raise ValueError(f"km must have shape [B, H, D] = {(b, h, d)}, got {tuple(km.shape)}")
    return km.contiguous()


def k_mean(k: torch.Tensor, tensor_layout: str = "HND") -> torch.Tensor:
    """k.mean(dim=seq) as [B, H, D] in k's dtype (fp32 accumulation, fixed order), on the GPU."""
    L = _lib.load()
    b, l, h, d = _dims(k, tensor_layout)
    out = torch.empty((b, h, d), dtype=k.dtype, device=k.device)
    ws = torch.empty(L.qattn_seq_mean_workspace_size(b, l, h, d), dtype=torch.uint8, device=k.device)
    _lib.check(L.qattn_seq_mean(_lib.seq(k, tensor_layout), _lib.dtype_code(k.dtype), b, l, h, d, _lib.ptr(out),
                                _lib.ptr(ws), ws.numel(), _lib.stream_of(k)))
    return out


def per_block_int8(q: torch.Tensor, k: torch.Tensor, km: Optional[torch.Tensor] = None, BLKQ: int = 128,
                   BLKK: int = 64, sm_scale: Optional[float] = None, tensor_layout: str = "HND",
                   variant: str = "cuda"):
    """Per-block INT8 quantization of q (sm_scale*1.44269504 folded in) and k (km subtracted).

    Same contract as tf_kernel.sageattn2.per_block_int8 (sageattn2.py:96-187); ``variant="triton"``
    reproduces the Triton quantizer (triton/quant_per_block.py:22-166) instead of the CUDA one.
    Returns (q_int8, q_scale [B, Hq, ceil(Lq/BLKQ)], k_int8, k_scale [B, Hkv, ceil(Lk/BLKK)]).
    """
    L = _lib.load()
    if q.dtype != k.dtype:
        raise ValueError("q and k must have the same dtype")
    b, lq, hq, d = _dims(q, tensor_layout)
    _, lk, hkv, _ = _dims(k, tensor_layout)
    q_int8 = torch.empty(q.shape, dtype=torch.int8, device=q.device)
    k_int8 = torch.empty(k.shape, dtype=torch.int8, device=k.device)
    q_scale = torch.empty((b, hq, (lq + BLKQ - 1) // BLKQ), dtype=torch.float32, device=q.device)
    k_scale = torch.empty((b, hkv, (lk + BLKK - 1) // BLKK), dtype=torch.float32, device=q.device)
    if sm_scale is None:
        sm_scale = d ** -0.5
    sm_scale *= LOG2E
    kmc = None if km is None else _mean_3d(km.to(k.dtype), b, hkv, d, tensor_layout)
    var = _lib.QATTN_QUANT_TRITON if variant == "triton" else _lib.QATTN_QUANT_CUDA
    _lib.check(L.qattn_quant_qk_per_block_int8(
        _lib.seq(q, tensor_layout), _lib.seq(k, tensor_layout), _lib.dtype_code(q.dtype), b, lq, lk, hq, hkv, d,
        _lib.ptr(kmc), _lib.seq(q_int8, tensor_layout), _lib.seq(k_int8, tensor_layout), _lib.ptr(q_scale),
        _lib.ptr(k_scale), float(sm_scale), BLKQ, BLKK, var, _lib.stream_of(q)))
    return q_int8, q_scale, k_int8, k_scale


def per_warp_int8(q: torch.Tensor, k: torch.Tensor, km: Optional[torch.Tensor] = None, BLKQ: int = 128,
                  WARPQ: int = 32, BLKK: int = 64, tensor_layout: str = "HND"):
    """sageattn2.per_warp_int8 (sageattn2.py:190-280): Q per WARPQ-row warp block (no sm_scale folded in),
    K per BLKK-row block after km.  Block shapes: (BLKQ, WARPQ, BLKK) = (128, 32, 64), the sm80/sm89
    kernels' tables, or (64, 16, 128), the sm90 entry's (sageattn2.py:1608-1611).  Returns (q_int8,
    q_scale [B, Hq, ceil(Lq/BLKQ)*4], k_int8, k_scale [B, Hkv, ceil(Lk/BLKK)])."""
    shapes = {(128, 32, 64): False, (64, 16, 128): True}
    if (BLKQ, WARPQ, BLKK) not in shapes:
        raise ValueError("per_warp_int8 supports (BLKQ, WARPQ, BLKK) = (128, 32, 64) or (64, 16, 128)")
    return _quant_gran(q, k, km, tensor_layout, "qattn_quant_qk_per_warp_int8_ex", 4, 1, shapes[(BLKQ, WARPQ, BLKK)])


def per_thread_int8(q: torch.Tensor, k: torch.Tensor, km: Optional[torch.Tensor] = None, BLKQ: int = 128,
                    WARPQ: int = 32, BLKK: int = 64, WARPK: int = 64, sm_scale=None, tensor_layout: str = "HND"):
    """triton.quant_per_thread.per_thread_int8 (quant_per_thread.py:267-369): per-thread scale classes,
    scale = amax/127 + 1e-7, round half away, K = half-rounded (k - km); sm_scale is not folded in.
    Block shapes: (BLKQ, WARPQ, BLKK, WARPK) = (128, 32, 64, 64) or the sm90 entry's (64, 16, 128, 128)
    (sageattn2.py:1614-1624).  Returns (q_int8, q_scale [B, Hq, ceil(Lq/BLKQ)*(BLKQ/WARPQ)*8], k_int8,
    k_scale [B, Hkv, ceil(Lk/BLKK)*4])."""
    shapes = {(128, 32, 64, 64): False, (64, 16, 128, 128): True}
    if (BLKQ, WARPQ, BLKK, WARPK) not in shapes:
        raise ValueError("per_thread_int8 supports (BLKQ, WARPQ, BLKK, WARPK) = (128, 32, 64, 64) or "
                         "(64, 16, 128, 128)")
    return _quant_gran(q, k, km, tensor_layout, "qattn_quant_qk_per_thread_int8_ex", 32, 4,
                       shapes[(BLKQ, WARPQ, BLKK, WARPK)])


def _scale_blocks(lq, lk, sm90):
    """Q and K scale blocks per (batch entry, head): 128-row Q / 64-row K blocks, or 64 / 128 (sm90)."""
    return (-(-lq // 64), -(-lk // 128)) if sm90 else (-(-lq // 128), -(-lk // 64))


def _quant_gran(q, k, km, tensor_layout, entry, q_per_blk, k_per_blk, sm90=False):
    L = _lib.load()
    if q.dtype != k.dtype:
        raise ValueError("q and k must have the same dtype")
    b, lq, hq, d = _dims(q, tensor_layout)
    _, lk, hkv, _ = _dims(k, tensor_layout)
    q_int8 = torch.empty(q.shape, dtype=torch.int8, device=q.device)
    k_int8 = torch.empty(k.shape, dtype=torch.int8, device=k.device)
    nqb, nkb = _scale_blocks(lq, lk, sm90)
    q_scale = torch.empty((b, hq, nqb * q_per_blk), dtype=torch.float32, device=q.device)
    k_scale = torch.empty((b, hkv, nkb * k_per_blk), dtype=torch.float32, device=q.device)
    kmc = None if km is None else _mean_3d(km.to(k.dtype), b, hkv, d, tensor_layout)
    _lib.check(getattr(L, entry)(
        _lib.seq(q, tensor_layout), _lib.seq(k, tensor_layout), _lib.dtype_code(q.dtype), b, lq, lk, hq, hkv, d,
        _lib.ptr(kmc), _lib.seq(q_int8, tensor_layout), _lib.seq(k_int8, tensor_layout), _lib.ptr(q_scale),
        _lib.ptr(k_scale), _lib.QATTN_SCALES_SM90 if sm90 else _lib.QATTN_SCALES_SM89, _lib.stream_of(q)))
    return q_int8, q_scale, k_int8, k_scale


def quant_per_block_int8(x: torch.Tensor, block_size: int, sm_scale: Optional[float] = None,
                         mean: Optional[torch.Tensor] = None, tensor_layout: str = "HND", variant: str = "cuda"):
    """One-tensor form: torch.ops.tf_kernel.quant_per_block_int8_cuda(_with_sm_scale / _fuse_sub_mean)
    (common_extension.cc:168-187).  ``sm_scale`` is multiplied as given (no log2e)."""
    L = _lib.load()
    b, l, h, d = _dims(x, tensor_layout)
    out = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    scale = torch.empty((b, h, (l + block_size - 1) // block_size), dtype=torch.float32, device=x.device)
    mc = None if mean is None else _mean_3d(mean.to(x.dtype), b, h, d, tensor_layout)
    var = _lib.QATTN_QUANT_TRITON if variant == "triton" else _lib.QATTN_QUANT_CUDA
    _lib.check(L.qattn_quant_per_block_int8(
        _lib.seq(x, tensor_layout), _lib.dtype_code(x.dtype), b, l, h, d, _lib.ptr(mc), _lib.seq(out, tensor_layout),
        _lib.ptr(scale), float(sm_scale or 0.0), int(sm_scale is not None), block_size, var, _lib.stream_of(x)))
    return out, scale


def per_channel_fp8(v: torch.Tensor, tensor_layout: str = "HND", scale_max: float = 448.0, smooth_v: bool = True):
    """V -> (v_fp8 [B, H, D, Lpad] float8_e4m3fn in tile layout, v_scale [B, H, D] fp32, vm).

    Same quantization as tf_kernel.sageattn2.per_channel_fp8 (sageattn2.py:320-407, MeanScaleKernel
    fused.cu:332-445), including the default ``smooth_v=True``: V minus its per-channel mean (sum over
    the tokens / tokens rounded up to 16) is quantized and ``vm`` [B, H, D] fp32 is returned (None when
    ``smooth_v`` is False).  The attention adds ``vm`` back (qattn_fwd(..., v_mean=vm))."""
    L = _lib.load()
    b, l, h, d = _dims(v, tensor_layout)
    lpad = (l + 63) // 64 * 64
    v_fp8 = torch.empty((b, h, d, lpad), dtype=torch.float8_e4m3fn, device=v.device)
    v_scale = torch.empty((b, h, d), dtype=torch.float32, device=v.device)
    vm = torch.empty((b, h, d), dtype=torch.float32, device=v.device) if smooth_v else None
    ws = torch.empty(L.qattn_per_channel_fp8_workspace_size(b, l, h, d), dtype=torch.uint8, device=v.device)
    _lib.check(L.qattn_per_channel_fp8_ex(_lib.seq(v, tensor_layout), _lib.dtype_code(v.dtype), b, l, h, d,
                                          float(scale_max), int(bool(smooth_v)), _lib.ptr(v_fp8), lpad,
                                          _lib.ptr(v_scale), _lib.ptr(vm), _lib.ptr(ws), ws.numel(),
                                          _lib.stream_of(v)))
    return v_fp8, v_scale, vm


def sage_quant(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str = "HND",
               qk_quant_gran: str = "per_block", sm_scale: Optional[float] = None, smooth_k: bool = True,
               scale_max: float = 448.0, smooth_v: bool = False, scale_layout: str = "sm89", quantize_q: bool = True):
    """The whole prologue of the INT8-QK / FP8-PV path in four launches (column passes of K and V,
    their finalize, V to FP8, K and Q to INT8): the same outputs, bit for bit, as k_mean + the
    per_block / per_warp / per_thread quantizer + per_channel_fp8 (CUDA quantizer variant).
    ``scale_layout="sm90"`` (per_warp / per_thread only) gives the sm90 entry's tables, as per_warp_int8 /
    per_thread_int8 with BLKQ=64, WARPQ=16, BLKK=128.  ``quantize_q=False`` leaves Q out (for qattn_fwd_q16,
    which quantizes it inside the attention kernel): q_int8 and q_scale are then None.
    Returns (q_int8, q_scale, k_int8, k_scale, km or None, v_fp8, v_scale, vm or None)."""
    L = _lib.load()
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k and v must have the same dtype")
    gran = {"per_block": 1, "per_warp": 2, "per_thread": 3}.get(qk_quant_gran)
    if gran is None:
        raise ValueError(f"unknown qk_quant_gran {qk_quant_gran!r}")
    if scale_layout not in ("sm89", "sm90"):
        raise ValueError(f"scale_layout must be 'sm89' or 'sm90', got {scale_layout!r}")
    sm90 = scale_layout == "sm90"
    if sm90 and gran == 1:
        raise ValueError("scale_layout='sm90' needs qk_quant_gran 'per_warp' or 'per_thread'")
    b, lq, hq, d = _dims(q, tensor_layout)
    _, lk, hkv, _ = _dims(k, tensor_layout)
    dev = q.device
    nqb, nkb = _scale_blocks(lq, lk, sm90)
    q_per = {1: 1, 2: 4, 3: 32}[gran]
    if quantize_q:
        q_int8 = torch.empty(q.shape, dtype=torch.int8, device=dev)
        q_scale = torch.empty((b, hq, nqb * q_per), dtype=torch.float32, device=dev)
    else:
        q_int8 = q_scale = None
    k_int8 = torch.empty(k.shape, dtype=torch.int8, device=dev)
    k_scale = torch.empty((b, hkv, nkb * (4 if gran == 3 else 1)), dtype=torch.float32, device=dev)
    km = torch.empty((b, hkv, d), dtype=k.dtype, device=dev) if smooth_k else None
    lpad = (lk + 63) // 64 * 64
    v_fp8 = torch.empty((b, hkv, d, lpad), dtype=torch.float8_e4m3fn, device=dev)
    v_scale = torch.empty((b, hkv, d), dtype=torch.float32, device=dev)
    vm = torch.empty((b, hkv, d), dtype=torch.float32, device=dev) if smooth_v else None
    ws = torch.empty(L.qattn_sage_quant_workspace_size(b, lk, hkv, d), dtype=torch.uint8, device=dev)
    if sm_scale is None:
        sm_scale = d ** -0.5
    _lib.check(L.qattn_sage_quant(
        _lib.seq(q, tensor_layout), _lib.seq(k, tensor_layout), _lib.seq(v, tensor_layout), _lib.dtype_code(q.dtype),
        b, lq if quantize_q else 0, lk, hq, hkv, d, gran + (2 if sm90 else 0), float(sm_scale * LOG2E),
        int(bool(smooth_k)), float(scale_max), int(bool(smooth_v)),
        _lib.seq(q_int8 if quantize_q else q, tensor_layout), _lib.ptr(q_scale), _lib.seq(k_int8, tensor_layout),
        _lib.ptr(k_scale), _lib.ptr(km), _lib.ptr(v_fp8), lpad, _lib.ptr(v_scale), _lib.ptr(vm), _lib.ptr(ws),
        ws.numel(), _lib.stream_of(q)))
    return q_int8, q_scale, k_int8, k_scale, km, v_fp8, v_scale, vm


def v_tile_half(v: torch.Tensor, tensor_layout: str = "HND") -> torch.Tensor:
    """V in the kernels' transposed tile layout, in its own dtype: [B, H, D, Lpad] (bf16/fp16 P.V path)."""
    L = _lib.load()
    b, l, h, d = _dims(v, tensor_layout)
    lpad = (l + 63) // 64 * 64
    v16 = torch.empty((b, h, d, lpad), dtype=v.dtype, device=v.device)
    _lib.check(L.qattn_v_tile_half(_lib.seq(v, tensor_layout), _lib.dtype_code(v.dtype), b, l, h, d, _lib.ptr(v16),
                                   lpad, _lib.stream_of(v)))
    return v16


def _kv_valid_tensor(kv_valid_len, b: int, device) -> Optional[torch.Tensor]:
    if kv_valid_len is None:
        return None
    t = torch.as_tensor(kv_valid_len, dtype=torch.int32)
    if t.dim() == 0:
        t = t.expand(b)
    if t.numel() != b:
        raise ValueError(f"kv_valid_len must have {b} entries")
    return t.to(device=device, dtype=torch.int32).contiguous()


_GRAN = {"per_block": _lib.QATTN_GRAN_BLOCK, "per_warp": _lib.QATTN_GRAN_WARP, "per_thread": _lib.QATTN_GRAN_THREAD}


def _check_attn_operands(q_int8, q_scale, k_int8, k_scale, v, v_scale, b, lq, lk, hq, hkv, d, gran, out, out_dtype,
                         sm90=False):
    """Shapes, dtypes and devices of qattn_fwd's operands: a scale tensor of another granularity or a V
    tile of the wrong size would make the kernel read outside them.  q_scale None: Q is half precision and
    quantized by the kernel (qattn_fwd_q16)."""
    nqb, nkb = _scale_blocks(lq, lk, sm90)
    q_per = {"per_block": 1, "per_warp": 4, "per_thread": 32}[gran]
    k_per = 4 if gran == "per_thread" else 1
    dev = q_int8.device
    q_dtypes = (torch.int8,) if q_scale is not None else (torch.bfloat16, torch.float16)
    if q_int8.dtype not in q_dtypes or k_int8.dtype != torch.int8:
        raise ValueError(f"q must be {' or '.join(str(t) for t in q_dtypes)} and k_int8 int8")
    scales = (("q_scale", q_scale, (b, hq, nqb * q_per)),) if q_scale is not None else ()
    for name, t, shape in scales + (("k_scale", k_scale, (b, hkv, nkb * k_per)),):
        if t.dtype != torch.float32 or tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 tensor of shape {shape} for qk_quant_gran="
                             f"{gran!r}, got {t.dtype} {tuple(t.shape)}")
    lpad = -(-lk // BLKK) * BLKK
    if v.dim() != 4 or tuple(v.shape[:3]) != (b, hkv, d) or v.shape[3] < lpad or v.shape[3] % BLKK or \
            not v.is_contiguous():
        raise ValueError(f"the V tile must be a contiguous [B, Hkv, D, Lpad] = [{b}, {hkv}, {d}, >= {lpad} (multiple "
                         f"of 64)] tensor from per_channel_fp8 / v_tile_half, got {tuple(v.shape)}")
    if v_scale is not None:
        if v.element_size() != 1:
            raise ValueError("with v_scale, V must be the e4m3 tile of per_channel_fp8")
        if v_scale.dtype != torch.float32 or tuple(v_scale.shape) != (b, hkv, d) or not v_scale.is_contiguous():
            raise ValueError(f"v_scale must be a contiguous float32 tensor of shape {(b, hkv, d)}, "
                             f"got {v_scale.dtype} {tuple(v_scale.shape)}")
    elif v.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("without v_scale, V must be the bf16 / fp16 tile of v_tile_half")
    if out is not None and (tuple(out.shape) != tuple(q_int8.shape) or out.dtype != out_dtype):
        raise ValueError(f"out must have q's shape {tuple(q_int8.shape)} and dtype {out_dtype}")
    for name, t in (("q_scale", q_scale), ("k_int8", k_int8), ("k_scale", k_scale), ("V", v), ("v_scale", v_scale),
                    ("out", out)):
        if t is not None and t.device != dev:
            raise ValueError(f"{name} is on {t.device}, q_int8 on {dev}")


def qattn_fwd(q_int8, q_scale, k_int8, k_scale, v_fp8, v_scale, *, tensor_layout="HND", out_dtype=torch.bfloat16,
              qk_mult=1.0, is_causal=False, q_offset=0, kv_valid_len=None, return_lse=False, num_splits=0,
              qk_quant_gran="per_block", out: Optional[torch.Tensor] = None, v_mean: Optional[torch.Tensor] = None,
              scale_layout: str = "sm89"):
    """Attention on already-quantized operands (the torch.ops.tf_kernel.qk_int8_sv_f8_accum_f32_fuse_v_scale
    _attn op, common_extension.cc:239-258).  With v_scale=None, v_fp8 is the half-dtype V tile from
    ``v_tile_half`` and P.V runs in that dtype (qk_int8_sv_f16_accum_f32_attn, common_extension.cc:214-218).
    ``qk_quant_gran`` names the layout of q_scale / k_scale ("per_block", "per_warp", "per_thread"); for
    the last two pass qk_mult = sm_scale * 1.44269504.  ``scale_layout="sm90"`` reads per-warp / per-thread
    tables of the sm90 block shapes (per_warp_int8 / per_thread_int8 with BLKQ=64, WARPQ=16, BLKK=128).
    Returns o (and the log2-domain LSE [B, Hq, Lq])."""
    L = _lib.load()
    b, lq, hq, d = _dims(q_int8, tensor_layout)
    _, lk, hkv, _ = _dims(k_int8, tensor_layout)
    if hq % hkv != 0:
        raise ValueError(f"num_qo_heads ({hq}) must be divisible by num_kv_heads ({hkv})")
    if qk_quant_gran not in _GRAN:
        raise ValueError(f"qk_quant_gran must be one of {sorted(_GRAN)}, got {qk_quant_gran!r}")
    if scale_layout not in ("sm89", "sm90"):
        raise ValueError(f"scale_layout must be 'sm89' or 'sm90', got {scale_layout!r}")
    sm90 = scale_layout == "sm90"
    if sm90 and qk_quant_gran == "per_block":
        raise ValueError("scale_layout='sm90' needs qk_quant_gran 'per_warp' or 'per_thread'")
    gran = _GRAN[qk_quant_gran] + (2 if sm90 else 0)
    _check_attn_operands(q_int8, q_scale, k_int8, k_scale, v_fp8, v_scale, b, lq, lk, hq, hkv, d, qk_quant_gran, out,
                         out_dtype, sm90)
    if v_mean is not None and (v_scale is None or v_mean.dtype != torch.float32 or
                               tuple(v_mean.shape) != (b, hkv, d) or not v_mean.is_contiguous()):
        raise ValueError(f"v_mean must be a contiguous float32 tensor of shape {(b, hkv, d)} (FP8 V only)")
    o = out if out is not None else torch.empty(q_int8.shape, dtype=out_dtype, device=q_int8.device)
    if v_scale is None:  # v_fp8 is then the half-dtype tile layout from v_tile_half
        v_kind = _lib.QATTN_V_BF16 if v_fp8.dtype == torch.bfloat16 else _lib.QATTN_V_FP16
    else:
        v_kind = _lib.QATTN_V_FP8
    lse = torch.empty((b, hq, lq), dtype=torch.float32, device=q_int8.device) if return_lse else None
    kvv = _kv_valid_tensor(kv_valid_len, b, q_int8.device)
    ns = num_splits if num_splits > 0 else L.qattn_fwd_ex_num_splits(b, lq, lk, hq, v_kind, gran)
    wsb = L.qattn_fwd_workspace_size(b, lq, hq, d, ns)
    ws = torch.empty(wsb, dtype=torch.uint8, device=q_int8.device) if wsb else None
    _lib.check(L.qattn_fwd_ex2(
        _lib.seq(q_int8, tensor_layout), _lib.ptr(q_scale), _lib.seq(k_int8, tensor_layout), _lib.ptr(k_scale),
        _lib.ptr(v_fp8), v_kind, v_fp8.shape[-1], _lib.ptr(v_scale), _lib.ptr(v_mean), _lib.seq(o, tensor_layout),
        _lib.dtype_code(o.dtype), b, lq, lk, hq, hkv, d, float(qk_mult), gran, int(bool(is_causal)), int(q_offset),
        _lib.ptr(kvv), _lib.ptr(lse), ns, _lib.ptr(ws), wsb, _lib.stream_of(q_int8)))
    return (o, lse) if return_lse else o


def qattn_fwd_q16(q, k_int8, k_scale, v_fp8, v_scale, *, tensor_layout="HND", qk_mult=1.0, is_causal=False,
                  q_offset=0, kv_valid_len=None, return_lse=False, num_splits=0, qk_quant_gran="per_thread",
                  out: Optional[torch.Tensor] = None, v_mean: Optional[torch.Tensor] = None):
    """Attention on half-precision Q (qattn_fwd_q16 in the C ABI): Q is quantized per thread (Triton rounding),
    per warp or per block (CUDA rounding) inside the attention kernel (the resident-K/V or the ping-pong
    kernel), bit-identical to per_thread_int8 / per_warp_int8 /
    per_block_int8 followed by qattn_fwd, without the int8 Q round trip through memory.  qk_mult is
    sm_scale * 1.44269504 for every granularity (per block it is multiplied into Q before quantization, as
    per_block_int8's sm_scale).  head_dim 128 for launches whose automatic kernel is one of those two, any
    launch with head_dim 64 (the ping-pong kernel's D = 64 form) (q16_supported).  Returns o (and the log2-domain LSE)."""
    L = _lib.load()
    b, lq, hq, d = _dims(q, tensor_layout)
    _, lk, hkv, _ = _dims(k_int8, tensor_layout)
    if hq % hkv != 0:
        raise ValueError(f"num_qo_heads ({hq}) must be divisible by num_kv_heads ({hkv})")
    if qk_quant_gran not in _GRAN:
        raise ValueError(f"qk_quant_gran must be one of {sorted(_GRAN)}, got {qk_quant_gran!r}")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("q must be bf16 or fp16")
    gran = _GRAN[qk_quant_gran]
    if not q16_supported(b, lq, lk, hq, d, qk_quant_gran, is_causal):
        raise ValueError(f"qattn_fwd_q16 does not cover this launch (head_dim {d}, {lq} x {lk}, causal={is_causal})")
    if v_scale is None:
        raise ValueError("qattn_fwd_q16 takes the e4m3 V tile and its v_scale")
    _check_attn_operands(q, None, k_int8, k_scale, v_fp8, v_scale, b, lq, lk, hq, hkv, d, qk_quant_gran, out, q.dtype)
    if v_mean is not None and (v_mean.dtype != torch.float32 or tuple(v_mean.shape) != (b, hkv, d) or
                               not v_mean.is_contiguous()):
        raise ValueError(f"v_mean must be a contiguous float32 tensor of shape {(b, hkv, d)}")
    o = out if out is not None else torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((b, hq, lq), dtype=torch.float32, device=q.device) if return_lse else None
    kvv = _kv_valid_tensor(kv_valid_len, b, q.device)
    ns = num_splits if num_splits > 0 else L.qattn_fwd_ex_num_splits(b, lq, lk, hq, _lib.QATTN_V_FP8, gran)
    wsb = L.qattn_fwd_workspace_size(b, lq, hq, d, ns)
    ws = torch.empty(wsb, dtype=torch.uint8, device=q.device) if wsb else None
    _lib.check(L.qattn_fwd_q16(
        _lib.seq(q, tensor_layout), _lib.seq(k_int8, tensor_layout), _lib.ptr(k_scale), _lib.ptr(v_fp8),
        v_fp8.shape[-1], _lib.ptr(v_scale), _lib.ptr(v_mean), _lib.seq(o, tensor_layout), _lib.dtype_code(q.dtype),
        b, lq, lk, hq, hkv, d, float(qk_mult), gran, int(bool(is_causal)), int(q_offset), _lib.ptr(kvv), _lib.ptr(lse),
        ns, _lib.ptr(ws), wsb, _lib.stream_of(q)))
    return (o, lse) if return_lse else o


def q16_supported(b, lq, lk, hq, d, qk_quant_gran, is_causal=False) -> bool:
    """Whether qattn_fwd_q16 (Q quantized inside the attention kernel) covers a launch of these sizes."""
    if qk_quant_gran not in _GRAN:
        return False
    return bool(_lib.load().qattn_fwd_q16_supported(b, lq, lk, hq, d, _GRAN[qk_quant_gran], int(bool(is_causal))))


def _pad_head_dim(x: torch.Tensor, native64: bool = False) -> torch.Tensor:
    """Zero-pad the head dimension to what the kernels take.  With ``native64`` (the FP8 P.V path, whose
    kernel has a head_dim-64 form) heads of at most 64 are padded to 64 and larger ones to 128, as the
    reference pads (sageattn2.py:1307-1316); otherwise every head is padded to 128."""
    d = x.size(-1)
    if d > 128:
        raise ValueError(f"Unsupported head_dim: {d}")
    target = 64 if native64 and d <= 64 else 128
    if d == target:
        return x
    return torch.nn.functional.pad(x, (0, target - d))


def _sage_forward(q, k, v, tensor_layout, is_causal, qk_quant_gran, sm_scale, pv_accum_dtype, smooth_k, smooth_v,
                  return_lse, kv_valid_len, q_offset, pv, quant_variant="cuda", sm90=False):
    dtype = q.dtype
    if not q.is_cuda:
        raise AssertionError("Input tensors must be on cuda.")
    if dtype not in (torch.float16, torch.bfloat16):
        raise AssertionError("Input tensors must be in dtype of torch.float16 or torch.bfloat16")
    if qk_quant_gran not in ("per_warp", "per_thread", "per_block"):
        raise AssertionError("qk_quant_gran must be either 'per_warp' or 'per_thread'.")
    if not (q.device == k.device == v.device):
        raise AssertionError("All tensors must be on the same device.")
    if not (q.dtype == k.dtype == v.dtype):
        raise AssertionError("All tensors must have the same dtype.")
    head_dim_og = q.size(-1)
    native64 = pv == "fp8"
    q, k, v = _pad_head_dim(q, native64), _pad_head_dim(k, native64), _pad_head_dim(v, native64)
    if not (q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1):
        raise AssertionError("Last dim of qkv must be contiguous.")
    if sm_scale is None:
        sm_scale = head_dim_og ** -0.5
    b, lq, hq, _ = _dims(q, tensor_layout)
    _, lk, hkv, _ = _dims(k, tensor_layout)
    if hq % hkv != 0:
        raise ValueError(f"num_qo_heads ({hq}) must be divisible by num_kv_heads ({hkv})")

    qk_mult = 1.0 if qk_quant_gran == "per_block" else sm_scale * LOG2E
    vm = None
    if pv == "fp8":
        # sageattn2.py:1368-1383: smooth_v only with "fp32" accumulation; "fp32+fp16" quantizes V to
        # |v8| <= 2.25 so that its fp16 tile partials cannot overflow (here P.V accumulates in fp32)
        if pv_accum_dtype not in ("fp32", "fp32+fp32", "fp32+fp16"):
            raise ValueError(f"pv_accum_dtype must be 'fp32', 'fp32+fp32' or 'fp32+fp16', got {pv_accum_dtype!r}")
        if pv_accum_dtype != "fp32" and smooth_v:
            warnings.warn(f"pv_accum_dtype is '{pv_accum_dtype}', smooth_v will be ignored.")
            smooth_v = False
        scale_max = 2.25 if pv_accum_dtype == "fp32+fp16" else 448.0
    if sm90:
        # the sm90 entry's quantizers and tables (sageattn2.py:1579-1660, V without smoothing), fused as
        # below: the same bits as k_mean + per_*_int8(BLKQ=64, WARPQ=16, BLKK=128) + per_channel_fp8
        q_int8, q_scale, k_int8, k_scale, km, v_fp8, v_scale, vm = sage_quant(
            q, k, v, tensor_layout=tensor_layout, qk_quant_gran=qk_quant_gran, sm_scale=sm_scale, smooth_k=smooth_k,
            scale_max=448.0, smooth_v=False, scale_layout="sm90")
    elif (pv == "fp8" and quant_variant == "cuda" and
          q16_supported(b, lq, lk, hq, q.size(-1), qk_quant_gran, is_causal)):
        # K mean, K INT8 and V FP8 in the fused prologue, Q quantized inside the attention kernel
        # (bit-identical to quantizing it first)
        _, _, k_int8, k_scale, km, v_fp8, v_scale, vm = sage_quant(
            q, k, v, tensor_layout=tensor_layout, qk_quant_gran=qk_quant_gran, sm_scale=sm_scale, smooth_k=smooth_k,
            scale_max=scale_max, smooth_v=smooth_v, quantize_q=False)
        res = qattn_fwd_q16(q, k_int8, k_scale, v_fp8, v_scale, tensor_layout=tensor_layout,
                            qk_mult=sm_scale * LOG2E, is_causal=is_causal, q_offset=q_offset, kv_valid_len=kv_valid_len,
                            return_lse=return_lse, qk_quant_gran=qk_quant_gran, v_mean=vm)
        return _sage_finish(res, q, km, hq, hkv, head_dim_og, tensor_layout, sm_scale, smooth_k, return_lse)
    elif pv == "fp8" and quant_variant == "cuda":
        # K mean, Q/K INT8 and V FP8 in one fused prologue (four launches)
        q_int8, q_scale, k_int8, k_scale, km, v_fp8, v_scale, vm = sage_quant(
            q, k, v, tensor_layout=tensor_layout, qk_quant_gran=qk_quant_gran, sm_scale=sm_scale, smooth_k=smooth_k,
            scale_max=scale_max, smooth_v=smooth_v)
    else:
        km = k_mean(k, tensor_layout) if smooth_k else None
        if qk_quant_gran == "per_block":
            q_int8, q_scale, k_int8, k_scale = per_block_int8(q, k, km, BLKQ, BLKK, sm_scale=sm_scale,
                                                              tensor_layout=tensor_layout, variant=quant_variant)
        else:  # sm_scale stays out of Q and is applied by the attention kernel (sm89 kernel :136,318-323)
            quant = per_thread_int8 if qk_quant_gran == "per_thread" else per_warp_int8
            q_int8, q_scale, k_int8, k_scale = quant(q, k, km, tensor_layout=tensor_layout)
        if pv == "fp8":
            v_fp8, v_scale, vm = per_channel_fp8(v, tensor_layout=tensor_layout, scale_max=scale_max,
                                                 smooth_v=smooth_v)
        else:
            if smooth_v:
                warnings.warn(f"pv_accum_dtype is '{pv_accum_dtype}', smooth_v will be ignored.")
            v_fp8, v_scale = v_tile_half(v, tensor_layout), None
    res = qattn_fwd(q_int8, q_scale, k_int8, k_scale, v_fp8, v_scale, tensor_layout=tensor_layout, out_dtype=dtype,
                    qk_mult=qk_mult, is_causal=is_causal, q_offset=q_offset, kv_valid_len=kv_valid_len,
                    return_lse=return_lse, qk_quant_gran=qk_quant_gran, v_mean=vm,
                    scale_layout="sm90" if sm90 else "sm89")
    return _sage_finish(res, q, km, hq, hkv, head_dim_og, tensor_layout, sm_scale, smooth_k, return_lse)


def _sage_finish(res, q, km, hq, hkv, head_dim_og, tensor_layout, sm_scale, smooth_k, return_lse):
    """Unpad O; natural-log LSE with the K-smoothing correction (sageattn2.py:1334-1354,1450-1455)."""
    o, lse = res if return_lse else (res, None)
    o = o[..., :head_dim_og]
    if not return_lse:
        return o
    lse = lse / LOG2E
    if smooth_k:
        # logits were computed against k - km: add back q.km * sm_scale
        qq = q if tensor_layout == "HND" else q.transpose(1, 2)
        kmb = km.repeat_interleave(hq // hkv, dim=1)  # [B, Hq, D]
        corr = torch.matmul(qq, kmb.unsqueeze(-1)).squeeze(-1).to(torch.float32)
        lse = lse + corr * sm_scale
    return o, lse


def sageattn_qk_int8_pv_fp8_cuda(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str = "HND",
                                 is_causal: bool = False, qk_quant_gran: str = "per_thread",
                                 sm_scale: Optional[float] = None, pv_accum_dtype: str = "fp32+fp16",
                                 smooth_k: bool = True, smooth_v: bool = False, return_lse: bool = False,
                                 kv_valid_len=None, q_offset: int = 0, **kwargs: Any):
    """INT8 Q.K^T + FP8 P.V attention (signature of sageattn2.py:1197-1210).

    Extra keyword arguments beyond the reference: ``kv_valid_len`` (int or per-batch sequence: keys at
    or beyond it are masked) and ``q_offset`` (causal diagonal offset, kv > q + q_offset is masked).

    ``pv_accum_dtype="fp32+fp16"`` differs from the reference in its arithmetic: the reference sums each
    64-key tile's P.V as two k=32 MMAs rounded to fp16 before adding it to the fp32 O
    (attn_utils.cuh:886-953); here V is quantized with the same scale_max 2.25 but P.V accumulates in fp32
    throughout, so results agree to within that fp16 rounding, not bit for bit.
    """
    return _sage_forward(q, k, v, tensor_layout, is_causal, qk_quant_gran, sm_scale, pv_accum_dtype, smooth_k,
                         smooth_v, return_lse, kv_valid_len, q_offset, pv="fp8")


def sageattn_qk_int8_pv_fp8_cuda_sm90(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str = "HND",
                                      is_causal: bool = False, qk_quant_gran: str = "per_thread",
                                      sm_scale: Optional[float] = None, pv_accum_dtype: str = "fp32+fp32",
                                      smooth_k: bool = True, return_lse: bool = False, kv_valid_len=None,
                                      q_offset: int = 0, **kwargs: Any):
    """The reference's sm90 entry (sageattn2.py:1460-1697): INT8 Q.K^T with the sm90 scale tables
    (per_warp_int8 / per_thread_int8 with BLKQ=64, WARPQ=16, BLKK=128), per-channel FP8 V without
    smoothing, P.V accumulated in fp32 ("fp32+fp32", the only accumulation it takes: "fp32" raises
    NotImplementedError there and here).  Heads of at most 64 run at 64, larger ones at 128, as there.
    ``kv_valid_len`` / ``q_offset`` as in sageattn_qk_int8_pv_fp8_cuda."""
    if qk_quant_gran not in ("per_warp", "per_thread"):
        raise AssertionError("qk_quant_gran must be either 'per_warp' or 'per_thread'.")
    if pv_accum_dtype == "fp32":
        raise NotImplementedError("Please use pv_accum_dtype='fp32+fp32' for sm90.")
    if pv_accum_dtype != "fp32+fp32":
        raise ValueError(f"pv_accum_dtype must be 'fp32+fp32' for sm90, got {pv_accum_dtype!r}")
    return _sage_forward(q, k, v, tensor_layout, is_causal, qk_quant_gran, sm_scale, pv_accum_dtype, smooth_k,
                         False, return_lse, kv_valid_len, q_offset, pv="fp8", sm90=True)


def sageattn_qk_int8_pv_fp16_cuda(q, k, v, tensor_layout: str = "HND", is_causal: bool = False,
                                  qk_quant_gran: str = "per_thread", sm_scale: Optional[float] = None,
                                  pv_accum_dtype: str = "fp32", smooth_k: bool = True, smooth_v: bool = False,
                                  return_lse: bool = False, kv_valid_len=None, q_offset: int = 0, **kwargs: Any):
    """INT8 Q.K^T + half-precision P.V (reference SAGE_ATTN_2_8_16 entry, sageattn2.py:930-1194): P is
    rounded to V's dtype and multiplied with V unquantized, accumulating in fp32."""
    return _sage_forward(q, k, v, tensor_layout, is_causal, qk_quant_gran, sm_scale, pv_accum_dtype, smooth_k,
                         smooth_v, return_lse, kv_valid_len, q_offset, pv="half")


def sageattn_qk_int8_pv_fp16_triton(q, k, v, tensor_layout: str = "HND", quantization_backend: str = "triton",
                                    is_causal: bool = False, attn_mask=None, sm_scale: Optional[float] = None,
                                    smooth_k: bool = True, return_lse: bool = False, kv_valid_len=None,
                                    q_offset: int = 0, **kwargs: Any):
    """Reference Triton entry (sageattn2.py:551-769): per-block quantizer with the Triton rounding
    (``quantization_backend="triton"``) or the CUDA one (``"cuda"``), half-precision P.V."""
    variant = "triton" if quantization_backend == "triton" else "cuda"
    return _sage_forward(q, k, v, tensor_layout, is_causal, "per_block", sm_scale, "fp32", smooth_k, False,
                         return_lse, kv_valid_len, q_offset, pv="half", quant_variant=variant)


def sageattn_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                    cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int, is_causal: bool = False,
                    sm_scale: Optional[float] = None, smooth_k: bool = True, **kwargs: Any) -> torch.Tensor:
    """Packed variable-length attention (sageattn2.py:772-927): q [total_q, Hq, D], k/v [total_k, Hkv, D],
    sequence b spanning rows cu_seqlens[b] .. cu_seqlens[b + 1].

    Same math as the reference: K smoothed by the mean over all packed keys (a half-precision subtraction),
    per-sequence Q/K blocks of 128/64 rows quantized with the Triton rounding
    (quant_per_block_varlen.py:22-70), V in fp16 and P rounded to fp16 for P.V
    (attn_qk_int8_block_varlen.py:42-65; P.V accumulates in fp32 here).  ``is_causal`` masks per
    sequence, top-left aligned.  The whole batch is four launches (block offsets, Q/K quantizer, V tiles,
    attention) whose workgroups read the sequence tables on the device: the host never reads cu_seqlens,
    and sizes its buffers from the packed lengths and max_seqlen_q / max_seqlen_k alone.  The tables are
    expected to be valid as in the reference (start at 0, non-decreasing, within the packed tensors, every
    length at most its max_seqlen); the kernels clamp each sequence to the packed tensors and to
    max_seqlen, so a malformed table gives wrong rows but never an out-of-bounds access.  Rows of
    sequences without keys are zero.
    """
    dtype = q.dtype
    if not q.is_cuda:
        raise AssertionError("Input tensors must be on cuda.")
    if dtype not in (torch.float16, torch.bfloat16):
        raise AssertionError("Input tensors must be in dtype of torch.float16 or torch.bfloat16")
    if not (q.device == k.device == v.device == cu_seqlens_q.device == cu_seqlens_k.device):
        raise AssertionError("All tensors must be on the same device.")
    if not (q.dtype == k.dtype == v.dtype):
        raise AssertionError("All tensors must have the same dtype.")
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape:
        raise ValueError("q must be [total_q, Hq, D] and k/v [total_k, Hkv, D]")
    head_dim_og = q.size(-1)
    q, k, v = _pad_head_dim(q), _pad_head_dim(k), _pad_head_dim(v)
    if not (q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1):
        raise AssertionError("Last dim of qkv must be contiguous.")
    if not (cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous()):
        raise AssertionError("cu_seqlens_q and cu_seqlens_k must be contiguous.")
    if cu_seqlens_q.dim() != 1 or cu_seqlens_q.shape != cu_seqlens_k.shape or cu_seqlens_q.numel() < 2:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must both have batch_size + 1 entries")
    hq, hkv, d = q.shape[1], k.shape[1], q.shape[2]
    if hq % hkv != 0:
        raise ValueError(f"num_qo_heads ({hq}) must be divisible by num_kv_heads ({hkv})")
    max_seqlen_q, max_seqlen_k = int(max_seqlen_q), int(max_seqlen_k)
    if max_seqlen_q < 0 or max_seqlen_k < 0 or max_seqlen_q > q.shape[0] or max_seqlen_k > k.shape[0]:
        raise ValueError("max_seqlen_q / max_seqlen_k must lie within the packed tensors")
    if sm_scale is None:
        sm_scale = head_dim_og ** -0.5
    L = _lib.load()
    st = _lib.stream_of(q)
    dev = q.device
    bsz = cu_seqlens_q.numel() - 1
    out = torch.zeros((q.shape[0], hq, d), dtype=dtype, device=dev)
    if max_seqlen_q == 0 or max_seqlen_k == 0 or q.shape[0] == 0 or k.shape[0] == 0:
        return out[..., :head_dim_og]
    cq = cu_seqlens_q if cu_seqlens_q.dtype == torch.int32 else cu_seqlens_q.to(torch.int32)
    ck = cu_seqlens_k if cu_seqlens_k.dtype == torch.int32 else cu_seqlens_k.to(torch.int32)
    offs = torch.empty((5, bsz + 1), dtype=torch.int32, device=dev)  # sanitised tables, block offsets
    seq_q, seq_k, cu_qs, cu_ks, cu_vt = offs[0], offs[1], offs[2], offs[3], offs[4]
    tq, tk = q.shape[0], k.shape[0]
    _lib.check(L.qattn_varlen_offsets(_lib.ptr(cq), _lib.ptr(ck), bsz, tq, tk, max_seqlen_q, max_seqlen_k,
                                      _lib.ptr(seq_q), _lib.ptr(seq_k), _lib.ptr(cu_qs), _lib.ptr(cu_ks),
                                      _lib.ptr(cu_vt), st))
    cq, ck = seq_q, seq_k  # the kernels read the sanitised tables only
    # block counts are bounded by ceil(total / block) + batch_size, whatever the split into sequences
    nqblk = -(-q.shape[0] // BLKQ) + bsz
    nkblk = -(-k.shape[0] // BLKK) + bsz
    q4, k4, v4 = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)  # [1, total, H, D] views
    km = k_mean(k4, "NHD") if smooth_k else None  # mean over every packed key, as k.mean(dim=0)
    q8 = torch.empty((1,) + tuple(q.shape), dtype=torch.int8, device=dev)
    k8 = torch.empty((1,) + tuple(k.shape), dtype=torch.int8, device=dev)
    qsc = torch.empty((nqblk, hq), dtype=torch.float32, device=dev)
    ksc = torch.empty((nkblk, hkv), dtype=torch.float32, device=dev)
    _lib.check(L.qattn_quant_qk_varlen_int8(
        _lib.seq(q4, "NHD"), _lib.seq(k4, "NHD"), _lib.dtype_code(dtype), bsz, tq, tk, max_seqlen_q, max_seqlen_k, hq, hkv,
        d, _lib.ptr(km) if km is not None else None, _lib.ptr(cq), _lib.ptr(ck), _lib.ptr(cu_qs), _lib.ptr(cu_ks),
        _lib.seq(q8, "NHD"), _lib.seq(k8, "NHD"), _lib.ptr(qsc), _lib.ptr(ksc), sm_scale * LOG2E,
        _lib.QATTN_QUANT_TRITON, st))
    v16 = v4 if v4.dtype == torch.float16 else v4.to(torch.float16)  # the reference runs P.V in fp16
    lpad = nkblk * BLKK
    vt = torch.empty((1, hkv, d, lpad), dtype=torch.float16, device=dev)
    _lib.check(L.qattn_v_tile_half_varlen(_lib.seq(v16, "NHD"), _lib.QATTN_FP16, bsz, tk, max_seqlen_k, hkv, d,
                                          _lib.ptr(ck), _lib.ptr(cu_vt), _lib.ptr(vt), lpad, st))
    o4 = out.unsqueeze(0)
    _lib.check(L.qattn_fwd_varlen(
        _lib.seq(q8, "NHD"), _lib.ptr(qsc), _lib.seq(k8, "NHD"), _lib.ptr(ksc), _lib.ptr(vt), lpad,
        _lib.seq(o4, "NHD"), _lib.dtype_code(dtype), bsz, tq, tk, max_seqlen_q, max_seqlen_k, hq, hkv, d, 1.0,
        1 if is_causal else 0, _lib.ptr(cq), _lib.ptr(ck), _lib.ptr(cu_qs), _lib.ptr(cu_ks), _lib.ptr(cu_vt), st))
    return out[..., :head_dim_og]


def sageattn(q, k, v, tensor_layout: str = "HND", is_causal: bool = False, sm_scale: Optional[float] = None,
             return_lse: bool = False, **kwargs: Any):
    """Architecture dispatch of the reference (sageattn2.py:415-548): gfx950 always takes the
    INT8-QK / FP8-PV kernel with per-warp scales, as the reference's sm89 branch does (:530-542)."""
    kwargs.setdefault("qk_quant_gran", "per_warp")
    return sageattn_qk_int8_pv_fp8_cuda(q, k, v, tensor_layout=tensor_layout, is_causal=is_causal,
                                        sm_scale=sm_scale, pv_accum_dtype="fp32+fp32", return_lse=return_lse,
                                        **kwargs)


__all__ = [
    "sageattn_varlen",
    "per_block_int8",
    "per_warp_int8",
    "per_thread_int8",
    "quant_per_block_int8",
    "per_channel_fp8",
    "sage_quant",
    "k_mean",
    "qattn_fwd",
    "sageattn",
    "sageattn_qk_int8_pv_fp8_cuda",
    "sageattn_qk_int8_pv_fp8_cuda_sm90",
    "qattn_fwd_q16",
    "q16_supported",
    "sageattn_qk_int8_pv_fp16_cuda",
    "sageattn_qk_int8_pv_fp16_triton",
    "v_tile_half",
]
