"""Block-sparse INT8 attention: mirror of ``telefuser.ops.attention.sparse_sage.sparse_sageattn``.

Follows telefuser/ops/attention/sparse_sage.py:25-80 (K smoothing by the sequence mean, the Triton
per-block quantizer of telefuser/kernel/triton/quant_per_block.py, V in fp16) and the k_block_id skip
of telefuser/kernel/triton/sparse_int8_attn.py:22-280: a 128-row query block visits only the 64-key
tiles whose mask byte is non-zero.  Runs on the gfx950 kernels through ``qattn_fwd_block_sparse``.

Differences, deliberate: P.V accumulates in fp32 (the reference's tl.dot accumulates each tile in
fp16); the default mask (``mask_id=None``) covers every key tile (the reference sizes its default from
the head dimension).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from . import sageattn2 as sa


def sparse_sageattn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask_id: Optional[torch.Tensor] = None,
                    is_causal: bool = False, tensor_layout: str = "HND") -> torch.Tensor:
    """q/k/v: [B, H, L, D] (HND) or [B, L, H, D] (NHD); mask_id: [B, H_kv, ceil(Lq/128), ceil(Lk/64)]
    (non-zero = visit the tile; indexed by the KV head, as the reference kernel does).  Returns the
    output in q's layout and dtype."""
    L = _lib.load()
    if not q.is_cuda:
        raise AssertionError("Input tensors must be on cuda.")
    if q.dtype not in (torch.float16, torch.bfloat16) or not (q.dtype == k.dtype == v.dtype):
        raise AssertionError("q, k and v must all be float16 or all bfloat16")
    b, lq, hq, d = sa._dims(q, tensor_layout)
    _, lk, hkv, _ = sa._dims(k, tensor_layout)
    if d != 128:
        raise ValueError(f"sparse_sageattn supports head_dim 128, got {d}")
    if hq % hkv != 0:
        raise ValueError(f"num_qo_heads ({hq}) must be divisible by num_kv_heads ({hkv})")
    if is_causal and lq != lk:
        raise AssertionError("qo_len and kv_len must be equal for causal attention")
    nqb, nkb = (lq + 127) // 128, (lk + 63) // 64
    if mask_id is None:
        mask_id = torch.ones((b, hkv, nqb, nkb), dtype=torch.int8, device=q.device)
    if tuple(mask_id.shape) != (b, hkv, nqb, nkb):
        raise ValueError(f"mask_id must be [B, H_kv, Q_blocks, K_blocks] = {(b, hkv, nqb, nkb)}, "
                         f"got {tuple(mask_id.shape)}")
    mask = mask_id.to(device=q.device, dtype=torch.int8)
    if mask.stride(-1) != 1 or mask.stride(0) != hkv * mask.stride(1):
        mask = mask.contiguous()
    km = sa.k_mean(k, tensor_layout)
    q8, qs, k8, ks = sa.per_block_int8(q, k, km, sa.BLKQ, sa.BLKK, sm_scale=d ** -0.5, tensor_layout=tensor_layout,
                                       variant="triton")
    v16 = v if v.dtype == torch.float16 else v.to(torch.float16)  # the reference runs P.V in fp16
    vt = sa.v_tile_half(v16, tensor_layout)
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    ns = L.qattn_fwd_block_sparse_num_splits(b, lq, lk, hq)
    wsb = L.qattn_fwd_workspace_size(b, lq, hq, d, ns)
    ws = torch.empty(wsb, dtype=torch.uint8, device=q.device) if wsb else None
    _lib.check(L.qattn_fwd_block_sparse(
        _lib.seq(q8, tensor_layout), _lib.ptr(qs), _lib.seq(k8, tensor_layout), _lib.ptr(ks), _lib.ptr(vt),
        _lib.QATTN_FP16, vt.shape[-1], _lib.seq(o, tensor_layout), _lib.dtype_code(o.dtype), b, lq, lk, hq, hkv, d,
        1.0, int(bool(is_causal)), _lib.ptr(mask), mask.stride(1), mask.stride(2), None, ns, _lib.ptr(ws), wsb,
        _lib.stream_of(q)))
    return o


__all__ = ["sparse_sageattn"]
