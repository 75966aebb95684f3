"""ctypes binding of libqattn.so (the C ABI declared in include/qattn.h).

The library is built in-tree (telefuser_amd/lib/libqattn.so) by ``telefuser_amd.build`` /
``__graft_entry__.build()``.  There is no fallback: if the library or a GPU is missing, loading
raises, so the HIP kernels are always what runs.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libqattn.so")

QATTN_BF16 = 0
QATTN_FP16 = 1
QATTN_QUANT_CUDA = 0
QATTN_QUANT_TRITON = 1
QATTN_GRAN_BLOCK, QATTN_GRAN_WARP, QATTN_GRAN_THREAD = 1, 2, 3
QATTN_GRAN_WARP_SM90, QATTN_GRAN_THREAD_SM90 = 4, 5
QATTN_SCALES_SM89, QATTN_SCALES_SM90 = 0, 1
QATTN_V_FP8, QATTN_V_BF16, QATTN_V_FP16 = 0, 1, 2
QATTN_KERNEL_AUTO, QATTN_KERNEL_ONE_BLOCK, QATTN_KERNEL_MULTI_BLOCK, QATTN_KERNEL_PINGPONG = 0, 1, 2, 3
QATTN_KERNEL_RESIDENT = 4
KERNEL_NAMES = {QATTN_KERNEL_ONE_BLOCK: "qattn_fwd_kernel", QATTN_KERNEL_MULTI_BLOCK: "qattn_fwd_kernel (multi-block)",
                QATTN_KERNEL_PINGPONG: "qattn_fwd_pp_kernel", QATTN_KERNEL_RESIDENT: "qattn_fwd_res_kernel"}

EXPORTED = (
    "qattn_last_error",
    "qattn_version",
    "qattn_quant_per_block_int8",
    "qattn_quant_qk_per_block_int8",
    "qattn_seq_mean_workspace_size",
    "qattn_seq_mean",
    "qattn_per_channel_fp8_workspace_size",
    "qattn_per_channel_fp8",
    "qattn_fwd_workspace_size",
    "qattn_fwd_num_splits",
    "qattn_fwd_ex_blocks_per_workgroup",
    "qattn_fwd_ex_kernel",
    "qattn_set_kernel",
    "qattn_last_kernel",
    "qattn_fwd",
    "qattn_v_tile_half",
    "qattn_fwd_pv16",
    "qattn_sage_quant_workspace_size",
    "qattn_sage_quant",
    "qattn_varlen_offsets",
    "qattn_quant_qk_varlen_int8",
    "qattn_v_tile_half_varlen",
    "qattn_fwd_varlen",
)


class QattnSeq(ctypes.Structure):
    """struct qattn_seq: element (b, l, h, d) at data[b*sb + l*sl + h*sh + d]."""

    _fields_ = [("data", ctypes.c_void_p), ("sb", ctypes.c_int64), ("sl", ctypes.c_int64), ("sh", ctypes.c_int64)]


class QattnError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"qattn error {code}: {msg}")
        self.code = code


_lib = None


def load() -> ctypes.CDLL:
    """Load libqattn.so and declare its signatures.  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
                           " (or make -C telefuser_amd/csrc)")
    L = ctypes.CDLL(LIB_PATH)
    i64, i32, vp, f32, sz = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float, ctypes.c_size_t
    S = QattnSeq
    L.qattn_last_error.restype = ctypes.c_char_p
    L.qattn_version.restype = i32
    L.qattn_quant_per_block_int8.argtypes = [S, i32, i64, i64, i64, i64, vp, S, vp, f32, i32, i32, i32, vp]
    L.qattn_quant_qk_per_block_int8.argtypes = [S, S, i32, i64, i64, i64, i64, i64, i64, vp, S, S, vp, vp, f32, i32,
                                                i32, i32, vp]
    L.qattn_seq_mean_workspace_size.argtypes = [i64, i64, i64, i64]
    L.qattn_seq_mean_workspace_size.restype = sz
    L.qattn_seq_mean.argtypes = [S, i32, i64, i64, i64, i64, vp, vp, sz, vp]
    L.qattn_per_channel_fp8_workspace_size.argtypes = [i64, i64, i64, i64]
    L.qattn_per_channel_fp8_workspace_size.restype = sz
    L.qattn_per_channel_fp8.argtypes = [S, i32, i64, i64, i64, i64, f32, vp, i64, vp, vp, sz, vp]
    L.qattn_fwd_workspace_size.argtypes = [i64, i64, i64, i64, i32]
    L.qattn_fwd_workspace_size.restype = sz
    L.qattn_fwd_num_splits.argtypes = [i64, i64, i64, i64]
    L.qattn_fwd_num_splits.restype = i32
    L.qattn_fwd.argtypes = [S, vp, S, vp, vp, i64, vp, S, i32, i64, i64, i64, i64, i64, i64, f32, i32, i64, vp, vp,
                            i32, vp, sz, vp]
    L.qattn_v_tile_half.argtypes = [S, i32, i64, i64, i64, i64, vp, i64, vp]
    L.qattn_fwd_pv16.argtypes = [S, vp, S, vp, vp, i32, i64, S, i32, i64, i64, i64, i64, i64, i64, f32, i32, i64, vp,
                                 vp, i32, vp, sz, vp]
    L.qattn_v_fp8_cache_workspace_size.argtypes = [i64, i64, i64, i64, i64]
    L.qattn_v_fp8_cache_workspace_size.restype = sz
    L.qattn_v_fp8_cache_update.argtypes = [S, i32, i64, i64, i64, i64, i64, i64, i64, i64, f32, vp, vp, i64, vp, vp,
                                           sz, vp]
    L.qattn_quant_qk_per_warp_int8.argtypes = [S, S, i32, i64, i64, i64, i64, i64, i64, vp, S, S, vp, vp, vp]
    L.qattn_quant_qk_per_thread_int8.argtypes = [S, S, i32, i64, i64, i64, i64, i64, i64, vp, S, S, vp, vp, vp]
    L.qattn_fwd_q16_supported.argtypes = [i64, i64, i64, i64, i64, i32, i32]
    L.qattn_fwd_q16_supported.restype = i32
    L.qattn_fwd_q16.argtypes = [S, S, vp, vp, i64, vp, vp, S, i32, i64, i64, i64, i64, i64, i64, f32, i32, i32, i64, vp,
                                vp, i32, vp, sz, vp]
    L.qattn_quant_qk_per_warp_int8_ex.argtypes = [S, S, i32, i64, i64, i64, i64, i64, i64, vp, S, S, vp, vp, i32, vp]
    L.qattn_quant_qk_per_thread_int8_ex.argtypes = [S, S, i32, i64, i64, i64, i64, i64, i64, vp, S, S, vp, vp, i32,
                                                    vp]
    L.qattn_fwd_ex_num_splits.argtypes = [i64, i64, i64, i64, i32, i32]
    L.qattn_fwd_ex_num_splits.restype = i32
    L.qattn_fwd_ex_blocks_per_workgroup.argtypes = [i64, i64, i64, i64, i32, i32, i32]
    L.qattn_fwd_ex_blocks_per_workgroup.restype = i32
    L.qattn_per_channel_fp8_ex.argtypes = [S, i32, i64, i64, i64, i64, f32, i32, vp, i64, vp, vp, vp, sz, vp]
    L.qattn_per_channel_fp8_ex.restype = i32
    L.qattn_fwd_ex2.argtypes = [S, vp, S, vp, vp, i32, i64, vp, vp, S, i32, i64, i64, i64, i64, i64, i64, f32, i32,
                                i32, i64, vp, vp, i32, vp, sz, vp]
    L.qattn_fwd_ex2.restype = i32
    L.qattn_fwd_noalloc_max_scratch.argtypes = []
    L.qattn_fwd_noalloc_max_scratch.restype = sz
    L.qattn_fwd_ex_noalloc.argtypes = [S, vp, S, vp, vp, i32, i64, vp, S, i32, i64, i64, i64, i64, i64, i64, f32, i32,
                                       i32, i64, vp, vp, i32, vp]
    L.qattn_fwd_ex_noalloc.restype = i32
    L.qattn_fwd_ex_kernel.argtypes = [i64, i64, i64, i64, i32, i32, i32, i32]
    L.qattn_fwd_ex_kernel.restype = i32
    L.qattn_set_kernel.argtypes = [i32]
    L.qattn_set_kernel.restype = i32
    L.qattn_last_kernel.argtypes = []
    L.qattn_last_kernel.restype = i32
    L.qattn_fwd_ex.argtypes = [S, vp, S, vp, vp, i32, i64, vp, S, i32, i64, i64, i64, i64, i64, i64, f32, i32, i32,
                               i64, vp, vp, i32, vp, sz, vp]
    L.qattn_fwd_block_sparse_num_splits.argtypes = [i64, i64, i64, i64]
    L.qattn_fwd_block_sparse_num_splits.restype = i32
    L.qattn_fwd_block_sparse.argtypes = [S, vp, S, vp, vp, i32, i64, S, i32, i64, i64, i64, i64, i64, i64, f32, i32,
                                         vp, i64, i64, vp, i32, vp, sz, vp]
    L.qattn_row_rstd.argtypes = [vp, i32, i64, i64, i64, f32, vp, vp]
    L.qattn_norm_rope_seq_mean.argtypes = [S, i32, i64, i64, i64, i64, vp, vp, vp, vp, i64, vp, vp, sz, vp]
    L.qattn_norm_rope_quant_qk.argtypes = [S, S, i32, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, i64, vp, S, S, vp,
                                           vp, f32, i32, vp]
    L.qattn_sage_quant_workspace_size.argtypes = [i64, i64, i64, i64]
    L.qattn_sage_quant_workspace_size.restype = sz
    L.qattn_sage_quant.argtypes = [S, S, S, i32, i64, i64, i64, i64, i64, i64, i32, f32, i32, f32, i32, S, vp, S, vp,
                                   vp, vp, i64, vp, vp, vp, sz, vp]
    L.qattn_sage_quant.restype = i32
    L.qattn_varlen_offsets.argtypes = [vp, vp, i64, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp]
    L.qattn_quant_qk_varlen_int8.argtypes = [S, S, i32, i64, i64, i64, i64, i64, i64, i64, i64, vp, vp, vp, vp, vp, S,
                                             S, vp, vp, f32, i32, vp]
    L.qattn_v_tile_half_varlen.argtypes = [S, i32, i64, i64, i64, i64, i64, vp, vp, vp, i64, vp]
    L.qattn_fwd_varlen.argtypes = [S, vp, S, vp, vp, i64, S, i32, i64, i64, i64, i64, i64, i64, i64, i64, f32, i32, vp,
                                   vp, vp, vp, vp, vp]
    for name in ("qattn_varlen_offsets", "qattn_quant_qk_varlen_int8", "qattn_v_tile_half_varlen",
                 "qattn_fwd_varlen"):
        getattr(L, name).restype = i32
    for name in ("qattn_row_rstd", "qattn_norm_rope_seq_mean", "qattn_norm_rope_quant_qk", "qattn_fwd_block_sparse", "qattn_quant_qk_per_warp_int8", "qattn_quant_qk_per_thread_int8", "qattn_fwd_ex",
                 "qattn_quant_qk_per_warp_int8_ex", "qattn_quant_qk_per_thread_int8_ex", "qattn_fwd_q16",
                 "qattn_v_fp8_cache_update", "qattn_quant_per_block_int8", "qattn_quant_qk_per_block_int8", "qattn_seq_mean",
                 "qattn_per_channel_fp8", "qattn_fwd", "qattn_v_tile_half", "qattn_fwd_pv16"):
        getattr(L, name).restype = i32
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != 0:
        msg = load().qattn_last_error().decode()
        if rc in (1, 5):
            raise ValueError(f"qattn error {rc}: {msg}")
        raise QattnError(rc, msg)


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def seq(t: torch.Tensor, layout: str) -> QattnSeq:
    """View a 4-D tensor as qattn_seq for "NHD" ([B, L, H, D]) or "HND" ([B, H, L, D])."""
    if t.stride(-1) != 1:
        raise ValueError("Last dim of qkv must be contiguous.")
    if layout == "NHD":
        return QattnSeq(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))
    if layout == "HND":
        return QattnSeq(t.data_ptr(), t.stride(0), t.stride(2), t.stride(1))
    raise ValueError(f"Unknown tensor layout: {layout}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return QATTN_BF16
    if dt == torch.float16:
        return QATTN_FP16
    raise ValueError("Input tensors must be in dtype of torch.float16 or torch.bfloat16")


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
