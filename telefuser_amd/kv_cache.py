"""Streaming self-attention against a rolling KV cache: the reference call site and an INT8-K cache.

The reference's streaming DiT (telefuser/models/lingbot_world_fast_dit.py:112-196) keeps a bf16 cache
dict ``{"k", "v": [B, size, H, D], "global_end_index", "local_end_index"}``.  Every call it

  1. rolls the non-sink part of the cache left when the new chunk does not fit (sink tokens stay),
  2. writes the new chunk's K/V at ``[local_end - n, local_end)``,
  3. runs ``attention()`` non-causally over the window ``[max(0, local_end - max_attention_size),
     local_end)`` - which re-quantizes the whole window (K mean, INT8 K, FP8 V) on every call.

``streaming_self_attention`` with such a dict reproduces that exactly (same index arithmetic, same
``attention()`` call).  ``QuantizedKVCache`` is the MI355X format of the same cache:

  * slots are a ring over the non-sink region: a roll moves a head offset instead of copying the
    cache, and non-causal attention does not depend on the order of its keys, so the attention
    window is the same *set* of keys as the reference's;
  * K is stored INT8 with per-64-slot block scales, smoothed by a mean frozen at the first write (any
    constant vector leaves the softmax unchanged); only the blocks that a write touches are
    re-quantized, from a bf16 copy of K in slot order;
  * V is stored FP8 (attention-kernel tile layout) with a running per-channel amax
    (``qattn_v_fp8_cache_update``): new rows are encoded with the current scale, and a (b, h) is
    re-encoded in full only when its amax grows;
  * a call then costs the quantization of the new rows plus the attention kernel, instead of
    re-quantizing the whole window.

Windows the ring cannot express as a prefix of slots (``max_attention_size`` smaller than the filled
cache, or re-running an older chunk after the ring wrapped) are served by gathering the window in the
reference's order from the bf16 copies and calling ``attention()``, i.e. with the reference's numerics.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib
from . import sageattn2 as sa
from .attention import AttentionConfig, AttnImplType, attention

BLK = sa.BLKK  # K quantization block (slots)


def _idx(x) -> int:
    return int(x.item()) if isinstance(x, torch.Tensor) else int(x)


def _roll_indices(n: int, size: int, sink: int, local_attn_size: int, current_start: int, global_end: int,
                  local_end: int):
    """Index arithmetic of lingbot_world_fast_dit.py:147-171.  Returns (evicted, new local_end)."""
    current_end = current_start + n
    if local_attn_size != -1 and current_end > global_end and n + local_end > size:
        evicted = n + local_end - size
        return evicted, local_end + current_end - global_end - evicted
    return 0, local_end + current_end - global_end


def streaming_self_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_cache, current_start: int, *,
                             sink_tokens: int = 0, local_attn_size: int = -1, max_attention_size: int = 1_000_000,
                             attention_config: AttentionConfig | None = None, **kwargs: Any) -> torch.Tensor:
    """One streaming step: cache update + attention of the new chunk's queries over the window.

    q, k, v: [B, n, H, D] (BSND), already normed and rotary-embedded.  ``kv_cache`` is the reference's
    dict (updated in place, exactly as lingbot_world_fast_dit.py:147-187 does) or a
    ``QuantizedKVCache``.  Returns [B, n, H, D].
    """
    if isinstance(kv_cache, QuantizedKVCache):
        return kv_cache.step(q, k, v, current_start, sink_tokens=sink_tokens, local_attn_size=local_attn_size,
                             max_attention_size=max_attention_size, **kwargs)
    if attention_config is None:
        attention_config = AttentionConfig(attn_impl=AttnImplType.SAGE_ATTN_2_8_8)
    n = q.shape[1]
    current_end = current_start + n
    cache_k, cache_v = kv_cache["k"], kv_cache["v"]
    size = cache_k.shape[1]
    global_end = _idx(kv_cache["global_end_index"])
    local_end = _idx(kv_cache["local_end_index"])
    evicted, new_local_end = _roll_indices(n, size, sink_tokens, local_attn_size, current_start, global_end,
                                           local_end)
    if evicted:
        rolled = local_end - evicted - sink_tokens
        src = slice(sink_tokens + evicted, sink_tokens + evicted + rolled)
        cache_k[:, sink_tokens:sink_tokens + rolled] = cache_k[:, src].clone()
        cache_v[:, sink_tokens:sink_tokens + rolled] = cache_v[:, src].clone()
    local_end = new_local_end
    local_start = local_end - n
    cache_k[:, local_start:local_end] = k
    cache_v[:, local_start:local_end] = v
    attn_start = max(0, local_end - max_attention_size)
    out = attention(q, cache_k[:, attn_start:local_end], cache_v[:, attn_start:local_end],
                    attention_config=attention_config, input_layout="BSND", output_layout="BSND", **kwargs)
    for key, val in (("global_end_index", current_end), ("local_end_index", local_end)):
        if isinstance(kv_cache[key], torch.Tensor):
            kv_cache[key].fill_(val)
        else:
            kv_cache[key] = val
    return out


class QuantizedKVCache:
    """Rolling KV cache holding INT8 K (block scales) and FP8 V (running per-channel scale) in ring order.

    ``size`` slots per (batch, head); ``sink_tokens`` slots at the front never roll.  Tensors:
      k16, v16   [B, size, H, D] input dtype, slot order (the source of every re-quantization)
      k8         [B, size, H, D] int8;  k_scale [B, H, ceil(size / 64)] fp32;  k_mean [B, H, D]
      v8         [B, H, D, Lpad] e4m3 tile layout;  v_scale, v_amax [B, H, D] fp32
    """

    def __init__(self, batch: int, size: int, heads: int, head_dim: int, *, sink_tokens: int = 0,
                 dtype: torch.dtype = torch.bfloat16, device: torch.device | str = "cuda"):
        if head_dim != 128:
            raise ValueError("QuantizedKVCache needs head_dim 128")
        if not 0 <= sink_tokens < size:
            raise ValueError("sink_tokens must lie in [0, size)")
        self.B, self.size, self.H, self.D, self.sink = batch, size, heads, head_dim, sink_tokens
        self.dtype, self.device = dtype, torch.device(device)
        shape = (batch, size, heads, head_dim)
        self.k16 = torch.zeros(shape, dtype=dtype, device=device)
        self.v16 = torch.zeros(shape, dtype=dtype, device=device)
        self.k8 = torch.zeros(shape, dtype=torch.int8, device=device)
        self.k_scale = torch.zeros((batch, heads, (size + BLK - 1) // BLK), dtype=torch.float32, device=device)
        self.k_mean: torch.Tensor | None = None
        self.lpad = (size + 63) // 64 * 64
        self.v8 = torch.zeros((batch, heads, head_dim, self.lpad), dtype=torch.float8_e4m3fn, device=device)
        self.v_scale = torch.zeros((batch, heads, head_dim), dtype=torch.float32, device=device)
        self.v_amax = torch.zeros((batch, heads, head_dim), dtype=torch.float32, device=device)
        self.global_end = 0
        self.local_end = 0
        self.head = 0        # ring offset of the non-sink region
        self.high_water = 0  # slots [0, high_water) hold data and are quantized

    # ---- slot mapping ----
    @property
    def ring(self) -> int:
        return self.size - self.sink

    def slot(self, pos: int) -> int:
        """Slot of reference cache position ``pos``."""
        if pos < self.sink:
            return pos
        return self.sink + (pos - self.sink + self.head) % self.ring

    def slot_ranges(self, begin: int, end: int) -> list[tuple[int, int]]:
        """Slot ranges (merged, in write order) holding reference positions [begin, end)."""
        out: list[tuple[int, int]] = []

        def add(a, b):
            if a >= b:
                return
            if out and out[-1][1] == a:
                out[-1] = (out[-1][0], b)
            else:
                out.append((a, b))

        if begin < self.sink:
            add(begin, min(end, self.sink))
        p = max(begin, self.sink)
        while p < end:
            s = self.slot(p)
            run = min(end - p, self.size - s)
            add(s, s + run)
            p += run
        return out

    def window_slots(self, begin: int, end: int) -> torch.Tensor:
        """Slot indices of reference positions [begin, end), in reference order."""
        pos = torch.arange(begin, end)
        ring_pos = self.sink + (pos - self.sink + self.head) % self.ring
        return torch.where(pos < self.sink, pos, ring_pos)

    # ---- one step ----
    def advance(self, k: torch.Tensor, v: torch.Tensor, current_start: int, local_attn_size: int = -1):
        """Host bookkeeping of one step: roll (ring head), write the chunk's bf16 rows into their slots.
        Returns (slot ranges written, new local_end).  Quantization is left to the caller."""
        n = k.shape[1]
        evicted, local_end = _roll_indices(n, self.size, self.sink, local_attn_size, current_start, self.global_end,
                                           self.local_end)
        local_start = local_end - n
        # positions the reference would leave stale (a gap before the new chunk) cannot be emulated
        defined_end = (self.local_end - evicted) if evicted else self.local_end
        if local_start < 0 or local_start > defined_end or local_end > self.size:
            raise ValueError("streaming step leaves a gap or runs outside the cache "
                             f"(local_start={local_start}, local_end={local_end}); use the dict cache")
        if evicted:
            if self.local_end - evicted - self.sink < 0:
                raise ValueError("eviction reaches into the sink tokens")
            self.head = (self.head + evicted) % self.ring
        self.local_end, self.global_end = local_end, current_start + n

        # write the chunk into its slots (bf16 copies), then re-quantize what the write touched
        ranges = self.slot_ranges(local_start, local_end)
        off = 0
        for a, e in ranges:
            self.k16[:, a:e] = k[:, off:off + e - a]
            self.v16[:, a:e] = v[:, off:off + e - a]
            off += e - a
        self.high_water = max(self.high_water, max(e for _, e in ranges))
        return ranges, local_end

    def step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, current_start: int, *, sink_tokens: int = 0,
             local_attn_size: int = -1, max_attention_size: int = 1_000_000, sm_scale: float | None = None,
             return_lse: bool = False, **kwargs: Any):
        if sink_tokens != self.sink:
            raise ValueError(f"cache was built for sink_tokens={self.sink}, got {sink_tokens}")
        b, n, hkv, d = k.shape
        if (b, hkv, d) != (self.B, self.H, self.D) or v.shape != k.shape:
            raise ValueError(f"k/v must be [{self.B}, n, {self.H}, {self.D}], got {tuple(k.shape)}, {tuple(v.shape)}")
        if q.shape[0] != b or q.shape[1] != n or q.shape[3] != d:
            raise ValueError("q must be [B, n, Hq, D] with the chunk length of k")
        if not (q.dtype == k.dtype == v.dtype == self.dtype):
            raise ValueError(f"q/k/v must be {self.dtype}")
        ranges, local_end = self.advance(k, v, current_start, local_attn_size)
        if self.k_mean is None:
            self.k_mean = sa.k_mean(k, "NHD")  # frozen smoothing vector
        self._requant_k(ranges)
        self._update_v(ranges)

        attn_start = max(0, local_end - max_attention_size)
        fast = attn_start == 0 and (self.head == 0 or local_end == self.size)
        if not fast:  # the reference's path on the window gathered in reference order
            idx = self.window_slots(attn_start, local_end).to(self.device)
            return attention(q, self.k16.index_select(1, idx), self.v16.index_select(1, idx),
                             attn_impl=AttnImplType.SAGE_ATTN_2_8_8, scale=sm_scale, return_lse=return_lse)
        return self._attend(q, local_end, sm_scale, return_lse)

    def _requant_k(self, ranges) -> None:
        L = _lib.load()
        hw = self.high_water
        for a, e in ranges:
            a0 = a // BLK * BLK
            e0 = min(-(-e // BLK) * BLK, hw)
            nblk = -(-(e0 - a0) // BLK)
            scale = torch.empty((self.B, self.H, nblk), dtype=torch.float32, device=self.device)
            src, dst = self.k16[:, a0:e0], self.k8[:, a0:e0]
            _lib.check(L.qattn_quant_per_block_int8(
                _lib.seq(src, "NHD"), _lib.dtype_code(self.dtype), self.B, e0 - a0, self.H, self.D,
                _lib.ptr(self.k_mean), _lib.seq(dst, "NHD"), _lib.ptr(scale), 0.0, 0, BLK, _lib.QATTN_QUANT_CUDA,
                _lib.stream_of(src)))
            self.k_scale[:, :, a0 // BLK:a0 // BLK + nblk] = scale

    def _update_v(self, ranges) -> None:
        L = _lib.load()
        for i in range(0, len(ranges), 2):
            (a0, e0), (a1, e1) = ranges[i], (ranges[i + 1] if i + 1 < len(ranges) else (0, 0))
            wsb = L.qattn_v_fp8_cache_workspace_size(self.B, e0 - a0, e1 - a1, self.H, self.D)
            ws = torch.empty(wsb, dtype=torch.uint8, device=self.device)
            _lib.check(L.qattn_v_fp8_cache_update(
                _lib.seq(self.v16, "NHD"), _lib.dtype_code(self.dtype), self.B, self.high_water, self.H, self.D,
                a0, e0, a1, e1, 448.0, _lib.ptr(self.v_amax), _lib.ptr(self.v8), self.lpad, _lib.ptr(self.v_scale),
                _lib.ptr(ws), wsb, _lib.stream_of(self.v16)))

    def _attend(self, q: torch.Tensor, n_valid: int, sm_scale: float | None, return_lse: bool):
        d = q.shape[-1]
        if sm_scale is None:
            sm_scale = d ** -0.5
        kv_valid = n_valid if n_valid < self.size else None
        b, lq, hq, _ = q.shape
        if sa.q16_supported(b, lq, self.k8.shape[1], hq, d, "per_block"):
            # the chunk's Q quantized per block inside the attention kernel (same bits as the quantizer below)
            res = sa.qattn_fwd_q16(q, self.k8, self.k_scale, self.v8, self.v_scale, tensor_layout="NHD",
                                   qk_mult=sm_scale * sa.LOG2E, kv_valid_len=kv_valid, return_lse=return_lse,
                                   qk_quant_gran="per_block")
        else:
            q8, qs = sa.quant_per_block_int8(q, sa.BLKQ, sm_scale=sm_scale * sa.LOG2E, tensor_layout="NHD")
            res = sa.qattn_fwd(q8, qs, self.k8, self.k_scale, self.v8, self.v_scale, tensor_layout="NHD",
                               out_dtype=q.dtype, kv_valid_len=kv_valid, return_lse=return_lse)
        if not return_lse:
            return res
        o, lse = res
        hq = q.shape[2]
        kmb = self.k_mean.repeat_interleave(hq // self.H, dim=1)  # [B, Hq, D]
        corr = torch.matmul(q.transpose(1, 2), kmb.unsqueeze(-1)).squeeze(-1).to(torch.float32)
        return o, lse / sa.LOG2E + corr * sm_scale


__all__ = ["streaming_self_attention", "QuantizedKVCache"]
