"""Front door mirroring ``telefuser.ops.attention.attention`` for the dense paths this backend serves.

Follows telefuser/ops/attention/attention_impl.py:112-315 (dense dispatch, BSND/BNSD handling, SDPA
fallback), telefuser/ops/attention/backends.py:87-150 (the ``sageattention`` module slot,
``SAGE_ATTN_AVAILABLE``, ``supports_return_lse``) and telefuser/core/config.py:117-221
(``AttnImplType``, ``AttentionConfig``).  The SAGE_* implementations run on this package's gfx950
kernels (``telefuser_amd.sageattn2``); TORCH_SDPA / TORCH_CUDNN stay torch's own kernels, and the
implementations this package does not provide (flash-attn, sparge, sparse) fall back to SDPA with a
one-time warning, as the reference does when a backend is missing.
"""

from __future__ import annotations

import logging
import os
from dataclasses import dataclass
from enum import Enum, auto
from typing import Any, Literal

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib

logger = logging.getLogger("telefuser_amd")


class AttnImplType(Enum):
    """Available attention implementations (same members as telefuser/core/config.py:117-132)."""

    TORCH_SDPA = auto()
    TORCH_CUDNN = auto()
    SAGE_ATTN_2_8_8 = auto()
    SAGE_ATTN_2_8_16 = auto()
    SAGE_ATTN_2_8_8_SM90 = auto()
    SPARGE_ATTN = auto()
    FLASH_ATTN_2 = auto()
    FLASH_ATTN_3 = auto()
    FLASH_ATTN_4 = auto()
    RADIAL_ATTN = auto()
    LOCAL_SPARSE_ATTN = auto()


@dataclass
class AttentionConfig:
    """Dense attention configuration (telefuser/core/config.py:161-221, sparse options omitted)."""

    attn_impl: AttnImplType = AttnImplType.TORCH_SDPA
    sparse_config: Any = None
    scale: float | None = None
    dropout: float = 0.0
    is_causal: bool = False

    @classmethod
    def dense_attention(cls, attn_impl: AttnImplType = AttnImplType.SAGE_ATTN_2_8_8, **kwargs: Any) -> "AttentionConfig":
        return cls(attn_impl=attn_impl, sparse_config=None, **kwargs)

    def is_sparse(self) -> bool:
        return self.attn_impl in (AttnImplType.RADIAL_ATTN, AttnImplType.LOCAL_SPARSE_ATTN)


# ---- backend slot (backends.py:87-99): the Sage module is this package's drop-in ----
SAGE_ATTN_AVAILABLE = os.path.exists(_lib.LIB_PATH)
SDPA_AVAILABLE = hasattr(F, "scaled_dot_product_attention")
if SAGE_ATTN_AVAILABLE:
    from . import sageattn2 as sageattention
else:  # pragma: no cover - only when the library was not built
    sageattention = None

_SAGE_IMPLS = (AttnImplType.SAGE_ATTN_2_8_8, AttnImplType.SAGE_ATTN_2_8_16, AttnImplType.SAGE_ATTN_2_8_8_SM90)
_BNSD_IMPLS = (AttnImplType.TORCH_CUDNN, AttnImplType.TORCH_SDPA, AttnImplType.SPARGE_ATTN)
_warned: set[str] = set()


def supports_return_lse(attn_impl: str) -> bool:
    """backends.py:137-150 for the implementations provided here."""
    return attn_impl in ("SAGE_ATTN_2_8_8", "SAGE_ATTN_2_8_16", "SAGE_ATTN_2_8_8_SM90") and SAGE_ATTN_AVAILABLE


def _warn_once(msg: str) -> None:
    if msg not in _warned:
        _warned.add(msg)
        logger.warning(msg)


def attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    attention_config: AttentionConfig | None = None,
    attn_impl: AttnImplType | None = None,
    attn_mask: Tensor | None = None,
    scale: float | None = None,
    input_layout: Literal["BSND", "BNSD"] = "BSND",
    output_layout: Literal["BSND", "BNSD"] = "BSND",
    is_causal: bool = False,
    return_lse: bool = False,
    kv_valid_len=None,
    **kwargs: Any,
) -> Tensor | tuple[Tensor, Tensor]:
    """Unified dense attention (attention_impl.py:112-315).

    q/k/v: [B, S, N, D] (BSND) or [B, N, S, D] (BNSD).  ``kv_valid_len`` (int or per-batch sequence) is
    this backend's key-padding mask for the SAGE implementations; as in the reference, ``attn_mask`` is
    not applied by the SAGE kernels (pass ``kv_valid_len`` instead) but is honoured by SDPA, and
    ``is_causal`` is not passed to the SAGE kernels (their output is non-causal; call
    ``sageattn2.sageattn_qk_int8_pv_fp8_cuda(..., is_causal=True)`` directly for causal SAGE attention).
    """
    if attention_config is None:
        attention_config = AttentionConfig(attn_impl=attn_impl or AttnImplType.TORCH_SDPA, scale=scale,
                                           is_causal=is_causal)
    impl = attention_config.attn_impl
    scale = scale if scale is not None else attention_config.scale
    is_causal = is_causal or attention_config.is_causal

    if impl in (AttnImplType.RADIAL_ATTN, AttnImplType.LOCAL_SPARSE_ATTN):
        _warn_once(f"Attention {impl} is not provided by telefuser_amd, falling back to TORCH_SDPA")
        impl = AttnImplType.TORCH_SDPA

    current = input_layout
    if input_layout == "BSND" and impl in _BNSD_IMPLS:
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
        current = "BNSD"
    elif input_layout == "BNSD" and impl not in _BNSD_IMPLS:
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
        current = "BSND"

    output = lse = None
    if impl in _SAGE_IMPLS and SAGE_ATTN_AVAILABLE:
        layout = "NHD" if current == "BSND" else "HND"
        fn = {
            AttnImplType.SAGE_ATTN_2_8_8: sageattention.sageattn_qk_int8_pv_fp8_cuda,
            AttnImplType.SAGE_ATTN_2_8_16: sageattention.sageattn_qk_int8_pv_fp16_cuda,
            AttnImplType.SAGE_ATTN_2_8_8_SM90: sageattention.sageattn_qk_int8_pv_fp8_cuda_sm90,
        }[impl]
        pv_accum = "fp32" if impl == AttnImplType.SAGE_ATTN_2_8_16 else "fp32+fp32"
        # is_causal is not forwarded: the reference's SAGE branch calls the sage functions without it
        # (attention_impl.py:249-283), so their output is non-causal whatever is_causal says
        result = fn(q, k, v, attn_mask=attn_mask, sm_scale=scale, tensor_layout=layout, pv_accum_dtype=pv_accum,
                    return_lse=return_lse, kv_valid_len=kv_valid_len, **kwargs)
        output, lse = result if return_lse else (result, None)
    elif impl in (AttnImplType.TORCH_SDPA, AttnImplType.TORCH_CUDNN) and SDPA_AVAILABLE:
        output = F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, scale=scale, is_causal=is_causal)

    if output is None:
        _warn_once(f"Attention {impl} not available, falling back to TORCH_SDPA")
        if current == "BSND":
            q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
            current = "BNSD"
        output = F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, scale=scale, is_causal=is_causal)

    if current != output_layout:
        output = output.transpose(1, 2).contiguous()
    if return_lse:
        return output, lse
    return output


__all__ = ["AttnImplType", "AttentionConfig", "attention", "supports_return_lse", "sageattention",
           "SAGE_ATTN_AVAILABLE"]
