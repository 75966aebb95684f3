"""ctypes front end of the CPU oracle (oracle/qattn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s
cpu_baseline leg as the checker.  The product package (``telefuser_amd``) never imports it.

All arrays are numpy; half-precision tensors are passed as their raw uint16 bit patterns.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

FP8_OFFSET = 8.807  # tf-kernel/csrc/sageattn2/qattn/attn_utils.cuh:35
LOG2E = 1.44269504  # constant the reference multiplies sm_scale by (sageattn2.py:177)


def build() -> str:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, vp, f32, i32, f64 = ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_int, ctypes.c_double
        L.oq_quant_per_block_int8.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, i64, vp, i64, i64, f32, i32,
                                              i64, vp, i64, i64, i64, vp]
        L.oq_quant_per_block_int8_triton.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, i64, vp, i64, i64, f32,
                                                     i64, vp, i64, i64, i64, vp]
        L.oq_per_channel_fp8.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, i64, f32, vp, i64, vp]
        L.oq_per_channel_fp8_ex.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, i64, f32, i32, vp, vp, vp, i64,
                                            vp]
        L.oq_qattn_fwd.argtypes = [vp, i64, i64, i64, vp, i64, vp, i64, i64, i64, vp, i64, vp, i64, vp, vp, i32,
                                   i64, i64, i64, i64, i64, i64, i64, i64, i64, f64, i32, i32, i64, vp, i64, i64,
                                   i64, i64, f64, i32, i32, i32, vp, i64, i64, vp, i32, i32, vp, vp]
        L.oq_norm_rope.argtypes = [vp, i32, i64, i64, i64, i64, vp, vp, vp, f32, vp]
        L.oq_quant_per_thread_int8.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, i64, vp, i64, i64, i32, vp,
                                               i64, i64, i64, vp]
        L.oq_quant_per_thread_int8_ex.argtypes = [vp, i32, i64, i64, i64, i64, i64, i64, i64, vp, i64, i64, i32,
                                                  i64, i64, vp, i64, i64, i64, vp]
        L.oq_attn_fp64.argtypes = [vp, vp, vp, i32, i64, i64, i64, i64, i64, i64, f64, i32, i64, vp, vp]
        L.oq_f32_to_e4m3.argtypes = [f32]
        L.oq_f32_to_e4m3.restype = ctypes.c_uint8
        L.oq_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.oq_e4m3_to_f32.restype = f32
        L.oq_f32_to_bf16.argtypes = [f32]
        L.oq_f32_to_bf16.restype = ctypes.c_uint16
        L.oq_f32_to_s8_rne_sat.argtypes = [f32]
        L.oq_f32_to_s8_rne_sat.restype = ctypes.c_int8
        L.oq_f32_to_s8_half_away.argtypes = [f32]
        L.oq_f32_to_s8_half_away.restype = ctypes.c_int8
        L.oq_num_threads.restype = i32
        L.oq_parallel_threads.restype = i32
        L.oq_set_threads.argtypes = [i32]
        L.oq_cvt_array.argtypes = [vp, i64, i32, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _bits(x: np.ndarray) -> np.ndarray:
    assert x.dtype == np.uint16, "half tensors are passed as uint16 bit patterns"
    return np.ascontiguousarray(x)


def _dims_nhd(x, layout):
    if layout == "NHD":
        B, L, H, D = x.shape
        sb, sl, sh = L * H * D, H * D, D
    else:
        B, H, L, D = x.shape
        sb, sh, sl = H * L * D, L * D, D
    return B, L, H, D, sb, sl, sh


def quant_per_block_int8(x_bits, km_bits=None, sm_scale=None, blk=128, layout="NHD", is_fp16=False,
                         variant="cuda"):
    """Quantize one tensor per block.  Returns (int8 tensor same layout, fp32 scale [B, H, nblk]).

    ``variant="cuda"`` follows QuantInt8Kernel (fused.cu:59-194); ``"triton"`` follows
    quant_per_block_int8_kernel (triton/quant_per_block.py:22-71).  ``sm_scale`` is the factor the
    kernel multiplies by (the callers pass sm_scale*1.44269504 for Q); None = no multiply.
    km_bits: [B, H, D] half bits (mean over the sequence) or None.
    """
    x_bits = _bits(x_bits)
    B, L, H, D, sb, sl, sh = _dims_nhd(x_bits, layout)
    out = np.zeros(x_bits.shape, np.int8)
    nblk = (L + blk - 1) // blk
    scale = np.zeros((B, H, nblk), np.float32)
    km_arr = None if km_bits is None else np.ascontiguousarray(km_bits.reshape(B, H, D))
    kmb, kmh = H * D, D
    if variant == "cuda":
        lib().oq_quant_per_block_int8(_p(x_bits), int(is_fp16), B, L, H, D, sb, sl, sh, _p(km_arr), kmb, kmh,
                                      float(sm_scale if sm_scale is not None else 0.0), int(sm_scale is not None),
                                      blk, _p(out), sb, sl, sh, _p(scale))
    else:
        lib().oq_quant_per_block_int8_triton(_p(x_bits), int(is_fp16), B, L, H, D, sb, sl, sh, _p(km_arr), kmb,
                                             kmh, float(sm_scale if sm_scale is not None else 1.0), blk, _p(out), sb,
                                             sl, sh, _p(scale))
    return out, scale


def norm_rope(x_bits, w_bits, cos, sin, head_dim, eps=1e-6, is_fp16=False):
    """RMSNorm over the last dim then interleaved RoPE per head (see oq_norm_rope).  x_bits [B, L, N]
    half bits, w_bits [N], cos/sin [L, head_dim/2] fp32.  Returns half bits [B, L, N]."""
    x_bits = np.ascontiguousarray(_bits(x_bits))
    B, L, N = x_bits.shape
    w = np.ascontiguousarray(_bits(w_bits))
    cs = np.ascontiguousarray(cos, dtype=np.float32)
    sn = np.ascontiguousarray(sin, dtype=np.float32)
    assert cs.shape == (L, head_dim // 2) and sn.shape == cs.shape and w.shape == (N,)
    out = np.zeros_like(x_bits)
    lib().oq_norm_rope(_p(x_bits), int(is_fp16), B, L, N, head_dim, _p(w), _p(cs), _p(sn), float(eps), _p(out))
    return out


def quant_per_thread_int8(x_bits, km_bits=None, is_key=False, layout="NHD", is_fp16=False, sm90=False):
    """Triton per-thread quantizer (triton/quant_per_thread.py:22-158,267-369).  Returns (int8 tensor same
    layout, fp32 scale [B, H, n]) with n = ceil(L/128)*32 for queries, ceil(L/64)*4 for keys; with
    ``sm90`` the sm90 entry's blocks (BLKQ 64, WARPQ 16, BLKK = WARPK 128; sageattn2.py:1614-1624):
    n = ceil(L/64)*32 for queries, ceil(L/128)*4 for keys."""
    x_bits = _bits(x_bits)
    B, L, H, D, sb, sl, sh = _dims_nhd(x_bits, layout)
    out = np.zeros(x_bits.shape, np.int8)
    if is_key:
        blk = 128 if sm90 else 64
        nblk = (L + blk - 1) // blk
    else:
        blkq, blk = (64, 16) if sm90 else (128, 32)
        nblk = (L + blkq - 1) // blkq * (blkq // blk)
    n = nblk * (4 if is_key else 8)
    scale = np.zeros((B, H, n), np.float32)
    km_arr = None if km_bits is None else np.ascontiguousarray(km_bits.reshape(B, H, D))
    lib().oq_quant_per_thread_int8_ex(_p(x_bits), int(is_fp16), B, L, H, D, sb, sl, sh, _p(km_arr), H * D, D,
                                      int(bool(is_key)), blk, nblk, _p(out), sb, sl, sh, _p(scale))
    return out, scale


def per_channel_fp8(v_bits, scale_max=448.0, layout="NHD", is_fp16=False, pad=64, smooth=False, mean_in=None):
    """V -> (e4m3 bytes [B, H, D, Lpad] in plain key order, v_scale [B, H, D]).  fused.cu:332-445.
    ``smooth=True`` is the sub_mean form and also returns the fp32 mean [B, H, D] (taken from ``mean_in``
    when given, else from a float64 sum); key slots past L are zero."""
    v_bits = _bits(v_bits)
    B, L, H, D, sb, sl, sh = _dims_nhd(v_bits, layout)
    Lpad = (L + pad - 1) // pad * pad
    v8 = np.zeros((B, H, D, Lpad), np.uint8)
    vs = np.zeros((B, H, D), np.float32)
    mean = np.zeros((B, H, D), np.float32)
    mi = None if mean_in is None else np.ascontiguousarray(mean_in, dtype=np.float32)
    lib().oq_per_channel_fp8_ex(_p(v_bits), int(is_fp16), B, L, H, D, sb, sl, sh, float(scale_max), int(smooth),
                                _p(mi), _p(mean), _p(v8), Lpad, _p(vs))
    return (v8, vs, mean) if smooth else (v8, vs)


def qattn_fwd(q8, q_scale, k8, k_scale, v8=None, v_scale=None, vh_bits=None, *, blkq=128, blkk=64,
              qk_mult=1.0, pv_mode=0, causal=False, q_offset=0, kv_valid=None, is_fp16=False, heads=None,
              qrows_limit=0, want_lse=False, tiles_per_split=0, lazy_tau=-1.0, lsum_rounded=False, q_gran=1,
              k_gran=1, tile_mask=None, v_mean=None, pv_f16_tile=False, p_linear=False):
    """Quantized attention in the reference's tile order.  q8/k8 NHD int8; returns fp32 O NHD
    (and log2-domain LSE [B, Hq, Lq] when want_lse).  lazy_tau >= 0 / tiles_per_split > 0 restate the
    device kernel's lazy running-max rule / KV-split schedule and lsum_rounded its row sum over the
    rounded P (defaults: the reference's schedule).  q_gran / k_gran: scale granularity codes of the reference
    (1 per block, 2 per warp, 3 per thread) - see oq_qattn_fwd.  tile_mask: int8 [B, Hkv, ceil(Lq/128),
    ceil(Lk/64)] block-sparse mask (0 = skip the key tile for that query block).  v_mean: fp32 [B, Hkv, D]
    added to the output (smoothed V).  pv_f16_tile: each tile's P.V summed as two 32-key fp16 MMAs before it
    joins the fp32 O (the reference's "fp32+fp16" accumulation).  p_linear (FP8 P.V only): P formed as the device
    kernels form it, the e4m3 byte RNE(8 (s - m - 0.057539) + 56) clamped to [0, 255], instead of e4m3(exp2(s - m))
    (see oq_qattn_fwd)."""
    q8 = np.ascontiguousarray(q8)
    k8 = np.ascontiguousarray(k8)
    B, Lq, Hq, D = q8.shape
    _, Lk, Hkv, _ = k8.shape
    out = np.zeros((B, Lq, Hq, D), np.float32)
    lse = np.full((B, Hq, Lq), np.nan, np.float32) if want_lse else None
    q_scale = np.ascontiguousarray(q_scale, dtype=np.float32)
    k_scale = np.ascontiguousarray(k_scale, dtype=np.float32)
    Lpad = 0
    if pv_mode == 0:
        v8 = np.ascontiguousarray(v8)
        v_scale = np.ascontiguousarray(v_scale, dtype=np.float32)
        Lpad = v8.shape[-1]
        vh_bits = None
    else:
        vh_bits = _bits(vh_bits)
    kvv = None if kv_valid is None else np.ascontiguousarray(np.asarray(kv_valid, np.int32))
    tm, tm_s1, tm_s2 = None, 0, 0
    if tile_mask is not None:
        tm = np.ascontiguousarray(tile_mask, dtype=np.int8)
        tm_s1, tm_s2 = tm.shape[2] * tm.shape[3], tm.shape[3]
    h0, h1 = (0, Hq) if heads is None else heads
    lib().oq_qattn_fwd(_p(q8), Lq * Hq * D, Hq * D, D, _p(q_scale), blkq, _p(k8), Lk * Hkv * D, Hkv * D, D,
                       _p(k_scale), blkk, _p(v8) if pv_mode == 0 else None, Lpad,
                       _p(v_scale) if pv_mode == 0 else None, _p(vh_bits), int(is_fp16), Lk * Hkv * D, Hkv * D, D,
                       B, Lq, Lk, Hq, Hkv, D, float(qk_mult), int(pv_mode), int(causal), int(q_offset), _p(kvv), h0,
                       h1, int(qrows_limit), int(tiles_per_split), float(lazy_tau), int(lsum_rounded), int(q_gran),
                       int(k_gran), _p(tm), tm_s1, tm_s2,
                       _p(None if v_mean is None else np.ascontiguousarray(v_mean, dtype=np.float32)),
                       int(bool(pv_f16_tile)), int(bool(p_linear)), _p(out), _p(lse))
    return (out, lse) if want_lse else out


def attn_fp64(q_bits, k_bits, v_bits, sm_scale, causal=False, q_offset=0, kv_valid=None, is_fp16=False):
    """Exact float64 softmax attention on half inputs (NHD), returned as fp32."""
    q_bits, k_bits, v_bits = _bits(q_bits), _bits(k_bits), _bits(v_bits)
    B, Lq, Hq, D = q_bits.shape
    _, Lk, Hkv, _ = k_bits.shape
    out = np.zeros((B, Lq, Hq, D), np.float32)
    kvv = None if kv_valid is None else np.ascontiguousarray(np.asarray(kv_valid, np.int32))
    lib().oq_attn_fp64(_p(q_bits), _p(k_bits), _p(v_bits), int(is_fp16), B, Lq, Lk, Hq, Hkv, D, float(sm_scale),
                       int(causal), int(q_offset), _p(kvv), _p(out))
    return out


def k_mean_bits(k_bits, layout="NHD"):
    """Per-(b, h, d) mean of K over the sequence in fp64, rounded to bf16 bits: [B, H, D]."""
    kf = bf16_bits_to_f32(k_bits).astype(np.float64)
    axis = 1 if layout == "NHD" else 2
    return f32_to_bf16_bits(kf.mean(axis=axis).astype(np.float32))


# ------------------------------------------------------------------------------------------------
# numpy helpers for half bit patterns
# ------------------------------------------------------------------------------------------------

def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def e4m3_to_f32(b: np.ndarray) -> np.ndarray:
    b = b.astype(np.int32)
    s = np.where(b >> 7, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e - 10.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return (s * v).astype(np.float32)


def cvt_array(x: np.ndarray, kind: str) -> np.ndarray:
    """Vectorised scalar conversions: kind in {"e4m3", "bf16", "s8_rne", "s8_half_away", "f16"}."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    code, dt = {"e4m3": (0, np.uint8), "bf16": (1, np.uint16), "s8_rne": (2, np.int8),
                "s8_half_away": (3, np.int8), "f16": (4, np.uint16)}[kind]
    out = np.zeros(x.shape, dt)
    lib().oq_cvt_array(_p(x), x.size, code, _p(out))
    return out


def num_threads() -> int:
    return lib().oq_num_threads()


def parallel_threads() -> int:
    """Threads that run an OpenMP parallel region of the oracle right now."""
    return lib().oq_parallel_threads()


def set_threads(n: int) -> None:
    lib().oq_set_threads(int(n))
