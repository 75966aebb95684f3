"""GPU parity of the quantized attention kernel.

Two oracles: (1) the CPU restatement of the reference's quantized math (oracle.qattn_fwd) fed with
the very int8 / fp8 tensors the GPU quantizers produced - isolates the attention kernel, gate
cosine >= 0.999 (observed ~0.99999); (2) float64 exact attention on the bf16 inputs - the north
star's end-to-end gate, cosine >= 0.999.  Max-abs errors are printed."""

import numpy as np
import pytest
import torch

from tests.gpu_util import log, lse_max_err, require_gpu, untile_v
from tests.inputs import bf16_bits, cosine, qkv

pytestmark = pytest.mark.gpu
COS_KERNEL = 0.99995  # same quantized operands and schedule: only exp2 ulps / fp32 sums differ
COS_E2E = 0.999
LOG2E = 1.44269504
KERNEL_LAZY_TAU = 3.0  # lazy running-max threshold of the FP8 / half attention kernels (kLazyTau in attn.hip)
# FP8 P.V kernels sum the e4m3-rounded P on the matrix pipe (row_sum_mfma in attn.hip); the oracle restates it
KERNEL_LSUM_ROUNDED = True
# FP8 P.V kernels form P without exp2: the e4m3 byte RNE(8 (s - m - 0.057539) + 56) (p_e4m3_x4 in attn.hip);
# the kernel-schedule oracle restates it (p_linear), the reference-schedule oracle keeps e4m3(exp2(s - m))
KERNEL_P_LINEAR = True
LSE_ROUNDED_SUM_BOUND = 0.0931  # log2(16/15): bound of the rounded-vs-unrounded row-sum LSE difference


GRAN_CODE = {"per_block": 1, "per_warp": 2, "per_thread": 3}
KERNEL_ONE_BLOCK, KERNEL_MULTI_BLOCK, KERNEL_PINGPONG, KERNEL_RESIDENT = 1, 2, 3, 4  # enum qattn_kernel


def _run_and_check(oracle, q, k, v, *, layout="NHD", causal=False, kv_valid=None, num_splits=0, q_offset=0,
                   check_truth=True, pv="fp8", gran="per_block", sm90=False):
    dev = require_gpu()
    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa

    B, Lq, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    log(f"attn B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} layout={layout} causal={causal} kv_valid={kv_valid} "
        f"splits={num_splits} gran={gran} pv={pv} D={D} sm90={sm90}")
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    if layout == "HND":
        qd, kd, vd = (t.transpose(1, 2).contiguous() for t in (qd, kd, vd))
    km = sa.k_mean(kd, layout)
    qk_mult = 1.0
    if gran == "per_block":
        q8, qs, k8, ks = sa.per_block_int8(qd, kd, km, sm_scale=D ** -0.5, tensor_layout=layout)
    else:
        quant = sa.per_thread_int8 if gran == "per_thread" else sa.per_warp_int8
        # the sm90 entry's block shapes (sageattn2.py:1608-1624)
        shapes = (dict(BLKQ=64, WARPQ=16, BLKK=128, **(dict(WARPK=128) if gran == "per_thread" else {}))
                  if sm90 else {})
        q8, qs, k8, ks = quant(qd, kd, km, tensor_layout=layout, **shapes)
        qk_mult = D ** -0.5 * sa.LOG2E
    gcode = GRAN_CODE[gran] + (2 if sm90 else 0)
    if pv == "fp8":
        v8, vs, _ = sa.per_channel_fp8(vd, tensor_layout=layout, smooth_v=False)
    else:
        v8, vs = sa.v_tile_half(vd, tensor_layout=layout), None
    o, lse = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, tensor_layout=layout, out_dtype=q.dtype, is_causal=causal,
                          q_offset=q_offset, kv_valid_len=kv_valid, num_splits=num_splits, return_lse=True,
                          qk_mult=qk_mult, qk_quant_gran=gran, scale_layout="sm90" if sm90 else "sm89")
    torch.cuda.synchronize()
    if layout == "HND":
        o, q8, k8 = o.transpose(1, 2), q8.transpose(1, 2), k8.transpose(1, 2)
    og = o.float().cpu().numpy()
    L = _lib.load()
    nkb = (Lk + 63) // 64
    v_kind = 0 if pv == "fp8" else (2 if q.dtype == torch.float16 else 1)
    ns = num_splits if num_splits > 0 else L.qattn_fwd_ex_num_splits(B, Lq, Lk, Hq, v_kind, gcode)
    ns = min(ns, nkb)
    tps = (nkb + ns - 1) // ns if ns > 1 else 0  # the GPU's KV-split schedule, restated on the CPU
    f16 = q.dtype == torch.float16
    vargs = (dict(v8=untile_v(v8), v_scale=vs.cpu().numpy()) if pv == "fp8"
             else dict(vh_bits=bf16_bits(v) if not f16 else v.contiguous().view(torch.int16).numpy().view(np.uint16),
                       pv_mode=1, is_fp16=f16))
    ref, ref_lse = oracle.qattn_fwd(q8.contiguous().cpu().numpy(), qs.cpu().numpy(), k8.contiguous().cpu().numpy(),
                                    ks.cpu().numpy(), **vargs, causal=causal, q_offset=q_offset,
                                    kv_valid=kv_valid, want_lse=True, tiles_per_split=tps,
                                    lazy_tau=KERNEL_LAZY_TAU, qk_mult=qk_mult, q_gran=gcode,
                                    k_gran=gcode, lsum_rounded=KERNEL_LSUM_ROUNDED and pv == "fp8",
                                    p_linear=KERNEL_P_LINEAR)
    c = cosine(og, ref)
    err = float(np.abs(og - ref).max())
    og_bhld = og.transpose(0, 2, 1, 3)  # rows in the LSE's [B, H, Lq] order
    lerr = lse_max_err(lse.cpu().numpy(), ref_lse, og_bhld)
    log(f"  vs quantized oracle (splits={ns}): cosine={c:.6f} max_abs={err:.4g} lse_max_abs={lerr:.3g}")
    assert c >= COS_KERNEL
    # the reference's own schedule (no split, eager running max) on the same quantized operands
    ref0, ref0_lse = oracle.qattn_fwd(q8.contiguous().cpu().numpy(), qs.cpu().numpy(),
                                      k8.contiguous().cpu().numpy(), ks.cpu().numpy(), **vargs, causal=causal,
                                      q_offset=q_offset, kv_valid=kv_valid, qk_mult=qk_mult, q_gran=gcode,
                                      k_gran=gcode, want_lse=True)
    c0 = cosine(og, ref0)
    lerr0 = lse_max_err(lse.cpu().numpy(), ref0_lse, og_bhld)
    log(f"  vs reference-schedule quantized math: cosine={c0:.6f} max_abs={float(np.abs(og - ref0).max()):.4g} "
        f"lse_max_abs={lerr0:.3g}")
    assert c0 >= COS_E2E
    assert lerr < 2e-2
    # The reference sums the unrounded p (accumulate_d); the FP8 kernels sum the e4m3-rounded P on the
    # matrix pipe.  Every p is rounded by a relative error of at most 2^-4, so the row sums differ by at
    # most a factor 1 / (1 - 2^-4) and the log2-domain LSE by at most log2(16/15) = 0.0931.
    assert lerr0 < LSE_ROUNDED_SUM_BOUND
    if check_truth:
        bits = (lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)) if f16 else bf16_bits
        truth = oracle.attn_fp64(bits(q), bits(k), bits(v), D ** -0.5, causal=causal,
                                 q_offset=q_offset, kv_valid=kv_valid, is_fp16=f16)
        ct = cosine(og, truth)
        log(f"  vs fp64 truth: cosine={ct:.6f} max_abs={float(np.abs(og - truth).max()):.4g}")
        assert ct >= COS_E2E
    return og


def test_config1_cpu_shape(oracle):
    q, k, v = qkv(1, 1024, 1024, 2, 2, seed=20250101, k_offset_std=0.5)
    _run_and_check(oracle, q, k, v)


@pytest.mark.parametrize("Lq,Lk", [(1000, 777), (130, 65), (64, 1), (257, 4000)])
def test_ragged_lengths(oracle, Lq, Lk):
    q, k, v = qkv(1, Lq, Lk, 2, 2, seed=Lq + Lk, k_offset_std=0.5)
    _run_and_check(oracle, q, k, v)


def test_hnd_layout_and_batch(oracle):
    q, k, v = qkv(2, 300, 500, 3, 3, seed=3, k_offset_std=1.0)
    _run_and_check(oracle, q, k, v, layout="HND")


def test_gqa(oracle):
    q, k, v = qkv(1, 384, 384, 8, 2, seed=4)
    _run_and_check(oracle, q, k, v)


def test_causal_top_left(oracle):
    q, k, v = qkv(1, 700, 700, 2, 2, seed=5)
    _run_and_check(oracle, q, k, v, causal=True)


def test_causal_with_offset_chunk(oracle):
    # a new chunk of 300 queries after 700 cached keys: query i sees keys <= i + 700
    q, k, v = qkv(1, 300, 1000, 2, 2, seed=6)
    _run_and_check(oracle, q, k, v, causal=True, q_offset=700)


def test_key_padding_cross_attention(oracle):
    # config-4 style: short K with per-batch valid lengths
    q, k, v = qkv(2, 512, 512, 4, 4, seed=7)
    k[0, 312:] = 0
    v[0, 312:] = 0
    k[1, 250:] = 0
    v[1, 250:] = 0
    _run_and_check(oracle, q, k, v, kv_valid=[312, 250])


@pytest.mark.parametrize("splits", [2, 5])
def test_kv_split_matches(oracle, splits):
    q, k, v = qkv(1, 256, 2000, 2, 2, seed=8, k_offset_std=0.5)
    _run_and_check(oracle, q, k, v, num_splits=splits)


def test_sageattn_api_and_lse(oracle):
    """Drop-in entry: NHD bf16 in, same shape out; LSE in natural log with the K-smoothing correction."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    q, k, v = qkv(1, 256, 384, 2, 2, seed=9, k_offset_std=1.0)
    o, lse = sa.sageattn_qk_int8_pv_fp8_cuda(q.to(dev), k.to(dev), v.to(dev), tensor_layout="NHD",
                                             pv_accum_dtype="fp32+fp32", return_lse=True)
    assert o.shape == q.shape and o.dtype == q.dtype and lse.shape == (1, 2, 256)
    s = torch.einsum("bqhd,bkhd->bhqk", q.double(), k.double()) * 128 ** -0.5
    want = torch.logsumexp(s, dim=-1).numpy()
    err = np.abs(lse.cpu().numpy() - want).max()
    log(f"lse max abs err {err:.4g}")
    assert err < 0.05
    truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(k), bf16_bits(v), 128 ** -0.5)
    assert cosine(o.float().cpu().numpy(), truth) >= COS_E2E


SM90_CASES = {
    # name: (B, Lq, Lk, Hq, Hkv, D, layout, causal, num_splits, gran, pv)
    "thread_ragged": (1, 200, 333, 2, 2, 128, "NHD", False, 0, "per_thread", "fp8"),
    "warp_ragged": (1, 200, 333, 2, 2, 128, "NHD", False, 0, "per_warp", "fp8"),
    "thread_short_q": (2, 40, 300, 2, 1, 128, "HND", False, 0, "per_thread", "fp8"),   # table < 128 rows
    "warp_causal": (1, 300, 300, 2, 2, 128, "NHD", True, 0, "per_warp", "fp8"),
    "thread_split": (1, 130, 2100, 2, 2, 128, "NHD", False, 3, "per_thread", "fp8"),
    "thread_d64": (1, 500, 700, 2, 2, 64, "NHD", False, 0, "per_thread", "fp8"),
    "thread_fp16_pv": (1, 300, 400, 4, 2, 128, "NHD", False, 0, "per_thread", "fp16"),
    "warp_many_blocks": (2, 1000, 1200, 4, 2, 128, "NHD", False, 0, "per_warp", "fp8"),
}


@pytest.mark.parametrize("case", sorted(SM90_CASES))
def test_sm90_scale_tables(oracle, case):
    """qattn_fwd reading the sm90 entry's scale tables (64-row Q blocks of 16-row warps, 128-key K blocks;
    sageattn2.py:1608-1624) against the oracle fed the same tables with q_gran / k_gran 4 or 5."""
    B, Lq, Lk, Hq, Hkv, D, layout, causal, ns, gran, pv = SM90_CASES[case]
    dt = torch.float16 if pv == "fp16" else torch.bfloat16
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, D=D, seed=31, k_offset_std=0.5, dtype=dt)
    _run_and_check(oracle, q, k, v, layout=layout, causal=causal, num_splits=ns, gran=gran, pv=pv, sm90=True)


@pytest.mark.parametrize("gran", ["per_warp", "per_thread"])
def test_sm90_entry(oracle, gran):
    """sageattn_qk_int8_pv_fp8_cuda_sm90 is the sm90 pipeline of the reference (sageattn2.py:1579-1697):
    K mean, the sm90-shape quantizers, V per channel without smoothing, attention on the sm90 tables.  Its
    output equals those steps run one by one, bit for bit, and float64 attention to the end-to-end bound;
    the LSE carries the q . k_mean correction.  "fp32" accumulation is refused as there."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    log(f"sm90 entry {gran}")
    q, k, v = qkv(1, 300, 500, 2, 2, seed=11, k_offset_std=0.5)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o90, lse = sa.sageattn_qk_int8_pv_fp8_cuda_sm90(qd, kd, vd, tensor_layout="NHD", qk_quant_gran=gran,
                                                    return_lse=True)
    km = sa.k_mean(kd, "NHD")
    shapes = dict(BLKQ=64, WARPQ=16, BLKK=128, **(dict(WARPK=128) if gran == "per_thread" else {}))
    quant = sa.per_thread_int8 if gran == "per_thread" else sa.per_warp_int8
    q8, qs, k8, ks = quant(qd, kd, km, tensor_layout="NHD", **shapes)
    v8, vs, _ = sa.per_channel_fp8(vd, tensor_layout="NHD", smooth_v=False)
    o = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, tensor_layout="NHD", out_dtype=q.dtype, qk_mult=128 ** -0.5 * LOG2E,
                     qk_quant_gran=gran, scale_layout="sm90")
    torch.cuda.synchronize()
    assert torch.equal(o90, o)
    truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(k), bf16_bits(v), 128 ** -0.5)
    assert cosine(o90.float().cpu().numpy(), truth) >= COS_E2E
    # natural-log LSE of the unsmoothed logits, against float64
    s = torch.einsum("bqhd,bkhd->bhqk", q.double(), k.double()) * 128 ** -0.5
    lse_ref = torch.logsumexp(s, dim=-1)
    assert (lse.double().cpu() - lse_ref).abs().max().item() < 0.1
    with pytest.raises(NotImplementedError):
        sa.sageattn_qk_int8_pv_fp8_cuda_sm90(qd, kd, vd, pv_accum_dtype="fp32")


@pytest.mark.parametrize("case", ["ragged", "gqa_hnd_padding", "causal_offset", "split", "per_thread",
                                  "per_warp_fp16"])
def test_head_dim_64_native(oracle, case):
    """head_dim 64 on the native D = 64 form of the ping-pong kernel (half the MFMA chain, 64-row V tiles),
    against the oracle on the same quantized operands and against float64 truth (through _run_and_check)."""
    from telefuser_amd import _lib

    kw = {}
    if case == "ragged":
        q, k, v = qkv(1, 1000, 777, 2, 2, D=64, seed=60, k_offset_std=0.5)
    elif case == "gqa_hnd_padding":
        q, k, v = qkv(2, 300, 1500, 4, 2, D=64, seed=61, k_offset_std=1.0)
        kw = dict(layout="HND", kv_valid=[1500, 700])
    elif case == "causal_offset":
        q, k, v = qkv(1, 500, 900, 2, 2, D=64, seed=62)
        kw = dict(causal=True, q_offset=400)
    elif case == "split":
        q, k, v = qkv(1, 520, 6000, 3, 3, D=64, seed=63, k_offset_std=0.5)
        kw = dict(num_splits=4, kv_valid=[5000])
    elif case == "per_thread":
        q, k, v = qkv(1, 700, 1300, 2, 1, D=64, seed=64, k_offset_std=0.5)
        kw = dict(gran="per_thread")
    else:
        q, k, v = qkv(1, 300, 400, 2, 2, D=64, seed=65, dtype=torch.float16)
        kw = dict(gran="per_warp")
    _run_and_check(oracle, q, k, v, **kw)
    assert _lib.load().qattn_last_kernel() == KERNEL_PINGPONG


@pytest.mark.parametrize("gran,causal,split", [("per_block", False, False), ("per_warp", True, False),
                                                ("per_thread", False, True), ("per_block", False, True)])
def test_fwd_q16_head_dim_64(gran, causal, split):
    """qattn_fwd_q16 on the head-dim-64 form of the ping-pong kernel (Q quantized inside it, NQF = 2 fragment
    columns per lane), unsplit and KV-split, bit-identical to the quantizer + qattn_fwd on the same K / V."""
    dev = require_gpu()
    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa

    B, Lq, Lk, Hq, Hkv = 1, 1000, 2400, 4, 2
    log(f"fwd_q16 head_dim 64: {gran} causal={causal} split={split}")
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, D=64, seed=66, k_offset_std=0.5)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    km = sa.k_mean(kd, "NHD")
    qk_mult = 64 ** -0.5 * LOG2E
    if gran == "per_block":
        q8, qs, k8, ks = sa.per_block_int8(qd, kd, km, sm_scale=64 ** -0.5, tensor_layout="NHD")
    else:
        quant = sa.per_thread_int8 if gran == "per_thread" else sa.per_warp_int8
        q8, qs, k8, ks = quant(qd, kd, km, tensor_layout="NHD")
    v8, vs, _ = sa.per_channel_fp8(vd, tensor_layout="NHD")
    assert sa.q16_supported(B, Lq, Lk, Hq, 64, gran, causal)
    kw = dict(tensor_layout="NHD", is_causal=causal, return_lse=True, qk_quant_gran=gran, num_splits=3 if split else 1)
    o_ref, l_ref = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, out_dtype=q.dtype,
                                qk_mult=1.0 if gran == "per_block" else qk_mult, **kw)
    o, l = sa.qattn_fwd_q16(qd, k8, ks, v8, vs, qk_mult=qk_mult, **kw)
    torch.cuda.synchronize()
    assert _lib.load().qattn_last_kernel() == KERNEL_PINGPONG
    assert torch.equal(o, o_ref), f"max diff {float((o.float() - o_ref.float()).abs().max())}"
    assert torch.equal(l, l_ref)


@pytest.mark.parametrize("d", [48, 64, 96])
def test_small_head_dims_through_the_drop_in(oracle, d):
    """sageattn_qk_int8_pv_fp8_cuda pads head_dim <= 64 to 64 (native kernel form) and 64 < D < 128 to 128, as
    sageattn2.py:1307-1316 does; the half-P.V entry pads to 128.  Output shape and accuracy against float64
    truth."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    q, k, v = qkv(1, 200, 300, 2, 2, D=d, seed=10 + d)
    truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(k), bf16_bits(v), d ** -0.5)
    for fn in (sa.sageattn_qk_int8_pv_fp8_cuda, sa.sageattn_qk_int8_pv_fp16_cuda):
        o = fn(q.to(dev), k.to(dev), v.to(dev), tensor_layout="NHD")
        assert o.shape == q.shape
        c = cosine(o.float().cpu().numpy(), truth)
        log(f"  head_dim {d} via {fn.__name__}: cos_truth={c:.6f}")
        assert c >= COS_E2E


def test_full_size_wan_480p_against_sdpa():
    """Config 2 at full size (L = 32760, H = 12): size-independent check against torch bf16 SDPA."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    g = torch.Generator(device=dev).manual_seed(1)
    q, k, v = (torch.randn((1, 32760, 12, 128), device=dev, generator=g, dtype=torch.bfloat16) for _ in range(3))
    log("full-size C2 shape vs SDPA")
    o = sa.sageattn_qk_int8_pv_fp8_cuda(q, k, v, tensor_layout="NHD")
    ref = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                                           v.transpose(1, 2)).transpose(1, 2)
    a, b = o.float().flatten(), ref.float().flatten()
    c = float((a @ b) / (a.norm() * b.norm()))
    log(f"  cosine vs SDPA {c:.6f}, max abs {float((a - b).abs().max()):.4g}")
    assert c >= 0.999
    assert torch.isfinite(o).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_half_pv_variant(oracle, dtype):
    """INT8 Q.K^T with P.V in the half dtype of V (the reference's SAGE_ATTN_2_8_16 / Triton math)."""
    q, k, v = qkv(1, 777, 1000, 2, 2, seed=12, k_offset_std=0.5, dtype=dtype)
    _run_and_check(oracle, q, k, v, pv="half")


def test_half_pv_causal_split_padding(oracle):
    q, k, v = qkv(2, 300, 1300, 2, 1, seed=13)
    _run_and_check(oracle, q, k, v, pv="half", num_splits=3, kv_valid=[1300, 900])
    _run_and_check(oracle, q, k[:, :300], v[:, :300], pv="half", causal=True)


def test_pv16_api_entry_points(oracle):
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    q, k, v = qkv(1, 256, 512, 2, 2, seed=14, dtype=torch.float16)
    truth = oracle.attn_fp64(*(t.contiguous().view(torch.int16).numpy().view(np.uint16) for t in (q, k, v)),
                             128 ** -0.5, is_fp16=True)
    for fn in (sa.sageattn_qk_int8_pv_fp16_cuda, sa.sageattn_qk_int8_pv_fp16_triton):
        o = fn(q.to(dev), k.to(dev), v.to(dev), tensor_layout="NHD")
        assert o.dtype == torch.float16 and o.shape == q.shape
        c = cosine(o.float().cpu().numpy(), truth)
        log(f"{fn.__name__}: cosine {c:.6f}")
        assert c >= 0.9995  # better than the FP8 P.V path: P and V are not rounded to e4m3


def test_attention_front_door_on_gpu(oracle):
    """telefuser-style attention() with the SAGE implementations, BSND and BNSD, against fp64 truth."""
    dev = require_gpu()
    from telefuser_amd import attention as A

    q, k, v = qkv(1, 300, 400, 2, 2, seed=15, k_offset_std=0.5)
    truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(k), bf16_bits(v), 128 ** -0.5)
    for impl in (A.AttnImplType.SAGE_ATTN_2_8_8, A.AttnImplType.SAGE_ATTN_2_8_16, A.AttnImplType.SAGE_ATTN_2_8_8_SM90):
        o = A.attention(q.to(dev), k.to(dev), v.to(dev), attn_impl=impl)
        assert cosine(o.float().cpu().numpy(), truth) >= COS_E2E
        ob = A.attention(*(t.to(dev).transpose(1, 2) for t in (q, k, v)), attn_impl=impl, input_layout="BNSD",
                         output_layout="BNSD")
        assert torch.equal(ob.transpose(1, 2).cpu(), o.cpu())


@pytest.mark.parametrize("gran", ["per_thread", "per_warp"])
@pytest.mark.parametrize("case", ["ragged", "gqa_hnd", "causal_offset", "padding", "split", "pv_bf16"])
def test_quant_granularities(oracle, gran, case):
    """The reference's default path: per-thread (Triton) or per-warp (CUDA) Q/K scales, sm_scale applied by
    the kernel (sageattn2.py:1356-1365), against the oracle on the same quantized operands and fp64 truth."""
    if case == "ragged":
        q, k, v = qkv(1, 333, 517, 2, 2, seed=31, k_offset_std=0.5)
        _run_and_check(oracle, q, k, v, gran=gran)
    elif case == "gqa_hnd":
        q, k, v = qkv(2, 260, 300, 4, 2, seed=32, k_offset_std=1.0)
        _run_and_check(oracle, q, k, v, gran=gran, layout="HND")
    elif case == "causal_offset":
        q, k, v = qkv(1, 200, 900, 2, 2, seed=33)
        _run_and_check(oracle, q, k, v, gran=gran, causal=True, q_offset=700)
    elif case == "padding":
        q, k, v = qkv(2, 300, 512, 2, 2, seed=34)
        _run_and_check(oracle, q, k, v, gran=gran, kv_valid=[400, 77])
    elif case == "split":
        q, k, v = qkv(1, 256, 3000, 2, 2, seed=35, k_offset_std=0.5)
        _run_and_check(oracle, q, k, v, gran=gran, num_splits=3)
    else:
        q, k, v = qkv(1, 300, 400, 2, 2, seed=36, k_offset_std=0.5)
        _run_and_check(oracle, q, k, v, gran=gran, pv="half")


@pytest.mark.parametrize("causal", [False, True])
def test_sageattn_varlen(oracle, causal):
    """Packed variable-length batch (sageattn2.py:772-927) in one device-side launch per stage: every
    sequence against the oracle (Triton quantizer, fp16 P.V, the kernel's schedule, no KV split) and
    float64 truth; sequences without queries or keys stay zero, and the host never reads cu_seqlens."""
    dev = require_gpu()
    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa

    lq = [100, 257, 0, 64, 70, 1] if not causal else [130, 257, 64, 300]
    lk = [130, 1100, 50, 64, 0, 700] if not causal else [130, 257, 64, 300]
    Hq, Hkv, D = 4, 2, 128
    cq, ck = np.concatenate([[0], np.cumsum(lq)]), np.concatenate([[0], np.cumsum(lk)])
    g = torch.Generator().manual_seed(41 + causal)
    q = torch.randn((int(cq[-1]), Hq, D), generator=g).to(torch.bfloat16)
    k = (torch.randn((int(ck[-1]), Hkv, D), generator=g) + 0.5).to(torch.bfloat16)
    v = torch.randn((int(ck[-1]), Hkv, D), generator=g).to(torch.bfloat16)
    log(f"varlen causal={causal} lq={lq} lk={lk}")
    L = _lib.load()
    L.qattn_set_kernel(_lib.QATTN_KERNEL_AUTO)
    o = sa.sageattn_varlen(q.to(dev), k.to(dev), v.to(dev), torch.tensor(cq, dtype=torch.int32, device=dev),
                           torch.tensor(ck, dtype=torch.int32, device=dev), max(lq), max(lk), is_causal=causal)
    torch.cuda.synchronize()
    assert L.qattn_last_kernel() == _lib.QATTN_KERNEL_ONE_BLOCK
    og = o.float().cpu().numpy()
    km = sa.k_mean(k.to(dev).unsqueeze(0), "NHD").cpu()  # [1, Hkv, D], the kernel's smoothing vector
    sm = D ** -0.5
    for b in range(len(lq)):
        rows = slice(int(cq[b]), int(cq[b + 1]))
        if lq[b] == 0:
            continue
        if lk[b] == 0:
            assert not og[rows].any()
            continue
        qb, kb, vb = q[rows].unsqueeze(0), k[int(ck[b]):int(ck[b + 1])].unsqueeze(0), v[int(ck[b]):int(ck[b + 1])].unsqueeze(0)
        q8, qs = oracle.quant_per_block_int8(bf16_bits(qb), sm_scale=sm * LOG2E, blk=128, variant="triton")
        k8, ks = oracle.quant_per_block_int8(bf16_bits(kb), km_bits=bf16_bits(km), blk=64, variant="triton")
        vh = vb.to(torch.float16).contiguous().view(torch.int16).numpy().view(np.uint16)
        ref = oracle.qattn_fwd(q8, qs, k8, ks, vh_bits=vh, pv_mode=1, is_fp16=True, causal=causal,
                               tiles_per_split=0, lazy_tau=KERNEL_LAZY_TAU)
        truth = oracle.attn_fp64(bf16_bits(qb), bf16_bits(kb), bf16_bits(vb), sm, causal=causal)
        got = og[rows][None]
        # the same kernel on this sequence alone, as a dense batch of one: bit-identical
        q8d, qsd = sa.quant_per_block_int8(qb.to(dev), 128, sm_scale=sm * LOG2E, tensor_layout="NHD",
                                           variant="triton")
        k8d, ksd = sa.quant_per_block_int8(kb.to(dev), 64, mean=km.to(dev), tensor_layout="NHD", variant="triton")
        vtd = sa.v_tile_half(vb.to(dev).to(torch.float16), "NHD")
        L.qattn_set_kernel(_lib.QATTN_KERNEL_ONE_BLOCK)
        try:
            od = sa.qattn_fwd(q8d, qsd, k8d, ksd, vtd, None, tensor_layout="NHD", out_dtype=torch.bfloat16,
                              is_causal=causal, num_splits=1)
        finally:
            L.qattn_set_kernel(_lib.QATTN_KERNEL_AUTO)
        assert torch.equal(od[0].cpu(), o[rows].cpu()), f"seq {b}: varlen launch differs from the dense launch"
        c, ct = cosine(got, ref), cosine(got, truth)
        err = float(np.abs(got - ref).max())
        log(f"  seq {b}: lq={lq[b]} lk={lk[b]} cos_oracle={c:.6f} cos_truth={ct:.6f} max|d|={err:.3g}")
        assert c >= COS_KERNEL
        assert ct >= COS_E2E


def test_sageattn_varlen_malformed_tables():
    """Sequence tables that break the contract (decreasing entries, entries past the packed tensors, a
    sequence longer than max_seqlen) are clamped on the device to disjoint row ranges of the packed
    tensors: the output equals the one computed from the clamped table written out by hand, and no
    access leaves the tensors."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    H, D, tq, tk = 2, 128, 700, 900
    g = torch.Generator().manual_seed(77)
    q = torch.randn((tq, H, D), generator=g).to(torch.bfloat16).to(dev)
    k = (torch.randn((tk, H, D), generator=g) + 0.5).to(torch.bfloat16).to(dev)
    v = torch.randn((tk, H, D), generator=g).to(torch.bfloat16).to(dev)
    # raw tables -> what the device makes of them (non-decreasing, clamped to [0, total])
    cases = [
        ([0, 300, 200, 700], [0, 400, 100, 900], [0, 300, 300, 700], [0, 400, 400, 900]),  # decreasing
        ([0, 100, 5000], [0, 300, 99999], [0, 100, 700], [0, 300, 900]),                  # past the end
        ([-50, 250, 700], [0, 450, 900], [0, 250, 700], [0, 450, 900]),                    # negative start
    ]
    for raw_q, raw_k, fix_q, fix_k in cases:
        mq = max(b - a for a, b in zip(fix_q, fix_q[1:]))
        mk = max(b - a for a, b in zip(fix_k, fix_k[1:]))
        t = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
        log(f"varlen malformed: q {raw_q} -> {fix_q}, k {raw_k} -> {fix_k}")
        o_raw = sa.sageattn_varlen(q, k, v, t(raw_q), t(raw_k), mq, mk)
        o_fix = sa.sageattn_varlen(q, k, v, t(fix_q), t(fix_k), mq, mk)
        torch.cuda.synchronize()
        assert torch.equal(o_raw, o_fix)
    # a sequence longer than max_seqlen_q: only its first max_seqlen_q rows are computed
    o_cut = sa.sageattn_varlen(q, k, v, t([0, 500, 700]), t([0, 450, 900]), 200, 450)
    o_ref = sa.sageattn_varlen(q, k, v, t([0, 200, 500, 700]), t([0, 450, 450, 900]), 200, 450)
    torch.cuda.synchronize()
    assert torch.equal(o_cut[:200], o_ref[:200]) and torch.equal(o_cut[500:700], o_ref[500:700])
    assert not o_cut[200:500].float().any()


@pytest.mark.parametrize("case", ["nhd", "hnd_gqa_causal", "split"])
def test_block_sparse(oracle, case):
    """sparse_sageattn (sparse_sage.py:25-80, sparse_int8_attn.py k_block_id skip) against the oracle with
    the same tile mask and against a float64 block-masked softmax; fully masked query blocks are zero."""
    dev = require_gpu()
    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa
    from telefuser_amd.sparse_sage import sparse_sageattn

    B, Lq, Lk, Hq, Hkv, layout, causal = {"nhd": (1, 300, 700, 2, 2, "NHD", False),
                                          "hnd_gqa_causal": (2, 384, 384, 4, 2, "HND", True),
                                          "split": (1, 128, 4000, 2, 2, "NHD", False)}[case]
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, seed=51, k_offset_std=0.5)
    nqb, nkb = (Lq + 127) // 128, (Lk + 63) // 64
    g = torch.Generator().manual_seed(52)
    mask = (torch.rand((B, Hkv, nqb, nkb), generator=g) < 0.5).to(torch.int8)
    mask[0, 0, 0] = 0  # a query block with no keys at all
    log(f"block-sparse {case}: density {float(mask.float().mean()):.2f}")
    args = [t.to(dev) for t in (q, k, v)]
    if layout == "HND":
        args = [t.transpose(1, 2).contiguous() for t in args]
    o = sparse_sageattn(*args, mask_id=mask.to(dev), is_causal=causal, tensor_layout=layout)
    torch.cuda.synchronize()
    if layout == "HND":
        o = o.transpose(1, 2)
    og = o.float().cpu().numpy()
    # oracle on the same quantized operands (Triton rounding, K smoothing), kernel schedule
    km = sa.k_mean(k.to(dev), "NHD").cpu()
    q8, qs = oracle.quant_per_block_int8(bf16_bits(q), sm_scale=128 ** -0.5 * LOG2E, blk=128, variant="triton")
    k8, ks = oracle.quant_per_block_int8(bf16_bits(k), km_bits=bf16_bits(km), blk=64, variant="triton")
    vh = v.to(torch.float16).contiguous().view(torch.int16).numpy().view(np.uint16)
    L = _lib.load()
    ns = min(L.qattn_fwd_block_sparse_num_splits(B, Lq, Lk, Hq), nkb)
    tps = (nkb + ns - 1) // ns if ns > 1 else 0
    ref = oracle.qattn_fwd(q8, qs, k8, ks, vh_bits=vh, pv_mode=1, is_fp16=True, causal=causal, tiles_per_split=tps,
                           lazy_tau=KERNEL_LAZY_TAU, tile_mask=mask.numpy())
    c = cosine(og, ref)
    # float64 truth with the block mask
    qf, kf, vf = (t.double().numpy() for t in (q, k, v))
    rep = Hq // Hkv
    truth = np.zeros_like(og, dtype=np.float64)
    for bb in range(B):
        for h in range(Hq):
            s = qf[bb, :, h] @ kf[bb, :, h // rep].T * 128 ** -0.5
            keep = np.repeat(np.repeat(mask[bb, h // rep].numpy().astype(bool), 128, 0), 64, 1)[:Lq, :Lk]
            if causal:
                keep &= np.tril(np.ones((Lq, Lk), bool))
            s = np.where(keep, s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            p = np.where(keep, np.exp(s - np.where(np.isfinite(mx), mx, 0)), 0)
            den = p.sum(axis=1, keepdims=True)
            truth[bb, :, h] = np.where(den > 0, (p @ vf[bb, :, h // rep]) / np.where(den > 0, den, 1), 0)
    ct = cosine(og, truth)
    log(f"  cos_oracle={c:.6f} cos_truth={ct:.6f} max_abs_truth={float(np.abs(og - truth).max()):.4g}")
    assert not og[0, :min(128, Lq), :rep].any()  # query block 0 of kv head 0 had no tiles
    assert c >= COS_KERNEL
    assert ct >= COS_E2E


@pytest.mark.parametrize("case", ["block_nhd_bf16", "thread_hnd_fp16"])
def test_multi_block_workgroups(oracle, case):
    """Short key ranges over a large grid run several query blocks per workgroup through one K/V pipeline.
    The per-block arithmetic is unchanged, so every head must match, bit for bit, a launch of a few heads
    (forced to one block per workgroup) on the same quantized operands; one (batch, head) is also checked
    against the oracle.  Covers key padding down to zero keys, a ragged last query block and the lse."""
    dev = require_gpu()
    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa

    gran, layout, dt = ("per_block", "NHD", torch.bfloat16) if case == "block_nhd_bf16" else \
        ("per_thread", "HND", torch.float16)
    B, Lq, Lk, H, D = 2, 16300, 600, 20, 128  # 10 key tiles: past the resident kernel
    kv_valid = [300, 0]
    L = _lib.load()
    qpw = L.qattn_fwd_ex_blocks_per_workgroup(B, Lq, Lk, H, 0, GRAN_CODE[gran], 0)
    log(f"multi-block {case}: B={B} Lq={Lq} Lk={Lk} H={H} kv_valid={kv_valid} blocks/workgroup={qpw}")
    assert qpw > 1
    assert L.qattn_fwd_ex_blocks_per_workgroup(1, 256, Lk, 2, 0, GRAN_CODE[gran], 0) == 1
    g = torch.Generator(device=dev).manual_seed(41)
    shape = (B, Lq, H, D) if layout == "NHD" else (B, H, Lq, D)
    kshape = (B, Lk, H, D) if layout == "NHD" else (B, H, Lk, D)
    q = torch.randn(shape, generator=g, device=dev).to(dt)
    k = (torch.randn(kshape, generator=g, device=dev) + 0.5).to(dt)
    v = torch.randn(kshape, generator=g, device=dev).to(dt)
    km = sa.k_mean(k, layout)
    qk_mult = 1.0
    if gran == "per_block":
        q8, qs, k8, ks = sa.per_block_int8(q, k, km, sm_scale=D ** -0.5, tensor_layout=layout)
    else:
        q8, qs, k8, ks = sa.per_thread_int8(q, k, km, tensor_layout=layout)
        qk_mult = D ** -0.5 * LOG2E
    v8, vs, _ = sa.per_channel_fp8(v, tensor_layout=layout, smooth_v=False)
    kw = dict(tensor_layout=layout, out_dtype=dt, kv_valid_len=kv_valid, return_lse=True, qk_mult=qk_mult,
              qk_quant_gran=gran)
    o, lse = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, **kw)
    assert L.qattn_last_kernel() == KERNEL_MULTI_BLOCK
    hd = 2 if layout == "NHD" else 1
    heads = [0, 7, 19]
    idx = torch.tensor(heads, device=dev)
    sel = lambda t, d: t.view(torch.uint8).index_select(d, idx).view(t.dtype) if t.dtype == torch.float8_e4m3fn \
        else t.index_select(d, idx).contiguous()
    prev = L.qattn_set_kernel(KERNEL_ONE_BLOCK)  # the reference launch: one query block per workgroup
    try:
        o3, lse3 = sa.qattn_fwd(sel(q8, hd), sel(qs, 1), sel(k8, hd), sel(ks, 1), sel(v8, 1), sel(vs, 1), **kw)
        assert L.qattn_last_kernel() == KERNEL_ONE_BLOCK
    finally:
        L.qattn_set_kernel(prev)
    torch.cuda.synchronize()
    assert torch.equal(sel(o, hd), o3), "multi-block output differs from the one-block-per-workgroup launch"
    assert torch.equal(sel(lse, 1), lse3)
    assert bool((o.select(0, 1) == 0).all()) and bool(torch.isneginf(lse[1]).all())
    # batch 0, head 7 against the oracle on the same quantized operands
    pick = lambda t: (t[:1, :, 7:8] if layout == "NHD" else t[:1, 7:8].transpose(1, 2)).contiguous().cpu().numpy()
    ref, ref_lse = oracle.qattn_fwd(pick(q8), qs[:1, 7:8].cpu().numpy(), pick(k8), ks[:1, 7:8].cpu().numpy(),
                                    v8=untile_v(v8[:1, 7:8]), v_scale=vs[:1, 7:8].cpu().numpy(),
                                    kv_valid=kv_valid[:1], want_lse=True, lazy_tau=KERNEL_LAZY_TAU, qk_mult=qk_mult,
                                    q_gran=GRAN_CODE[gran], k_gran=GRAN_CODE[gran], lsum_rounded=KERNEL_LSUM_ROUNDED,
                                    p_linear=KERNEL_P_LINEAR)
    og = pick(o.float())
    c = cosine(og, ref)
    log(f"  head 7 vs quantized oracle: cosine={c:.6f} max_abs={float(np.abs(og - ref).max()):.4g}")
    assert c >= COS_KERNEL
    assert float(np.max(np.abs(lse[:1, 7:8].cpu().numpy() - ref_lse))) < 2e-2


@pytest.mark.parametrize("case", ["padding", "ragged", "empty_batch", "gqa_hnd_thread", "fp16_warp_gqa", "one_tile",
                                  "tiny", "smooth_v", "many_blocks", "zero_scale_block"])
def test_resident_kernel_matches(oracle, case):
    """The resident-K/V kernel (whole key range in LDS, 12 barrier-free waves per workgroup, each on its own
    32-row query blocks) runs the per-element arithmetic of qattn_fwd_kernel, so output and LSE must be
    identical, bit for bit, on the same operands.  Checked with key padding (a tail tile of 44 keys), one
    batch without any valid key, ragged lengths whose last wave block is partial, GQA + HND + per-thread
    scales, GQA + per-warp scales + fp16 output, a single tile, fewer queries than one wave block,
    smoothed V (v_mean epilogue), enough query blocks that every wave walks many of them, and an
    all-zero query block under the Triton rounding (q_scale 0: the masked tail tile takes the per-logit
    select instead of -inf logits); the automatic rule must pick the kernel for these non-causal FP8
    launches with Lk <= 512, and the padding case is also checked against the oracle."""
    dev = require_gpu()
    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa

    B, Lq, Lk, Hq, Hkv, layout, kv_valid, gran = {
        "padding": (1, 1500, 512, 4, 4, "NHD", [300], "per_block"),
        "ragged": (2, 1001, 333, 3, 3, "NHD", None, "per_block"),
        "empty_batch": (2, 700, 450, 2, 2, "NHD", [450, 0], "per_block"),
        "gqa_hnd_thread": (1, 2000, 500, 4, 2, "HND", None, "per_thread"),
        "fp16_warp_gqa": (1, 900, 260, 6, 2, "NHD", None, "per_warp"),
        "one_tile": (1, 640, 64, 2, 2, "NHD", None, "per_block"),
        "tiny": (1, 31, 7, 1, 1, "NHD", None, "per_block"),
        "smooth_v": (1, 1200, 400, 2, 2, "NHD", [390], "per_block"),
        "many_blocks": (1, 40000, 300, 2, 2, "NHD", None, "per_block"),
        "zero_scale_block": (1, 1000, 400, 2, 2, "NHD", [300], "per_block"),
    }[case]
    log(f"resident vs one-block: {case} B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} layout={layout} "
        f"kv_valid={kv_valid} gran={gran}")
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, seed=4343, k_offset_std=0.5)
    if case == "zero_scale_block":
        q[:, :128, 0] = 0  # first query block of head 0: amax 0, q_scale 0 under the Triton rounding
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    if layout == "HND":
        qd, kd, vd = (t.transpose(1, 2).contiguous() for t in (qd, kd, vd))
    km = sa.k_mean(kd, layout)
    qk_mult = 1.0
    if gran == "per_block":
        variant = "triton" if case == "zero_scale_block" else "cuda"
        q8, qs, k8, ks = sa.per_block_int8(qd, kd, km, sm_scale=128 ** -0.5, tensor_layout=layout, variant=variant)
        if case == "zero_scale_block":
            assert float(qs[0, 0, 0]) == 0.0
    else:
        quant = sa.per_thread_int8 if gran == "per_thread" else sa.per_warp_int8
        q8, qs, k8, ks = quant(qd, kd, km, tensor_layout=layout)
        qk_mult = 128 ** -0.5 * LOG2E
    v8, vs, vm = sa.per_channel_fp8(vd, tensor_layout=layout, smooth_v=case == "smooth_v")
    out_dtype = torch.float16 if case == "fp16_warp_gqa" else torch.bfloat16
    kw = dict(tensor_layout=layout, out_dtype=out_dtype, is_causal=False, kv_valid_len=kv_valid,
              return_lse=True, qk_mult=qk_mult, qk_quant_gran=gran, num_splits=1, v_mean=vm)
    L = _lib.load()
    assert L.qattn_fwd_ex_kernel(B, Lq, Lk, Hq, 0, _lib.QATTN_GRAN_BLOCK, 0, 0) == KERNEL_RESIDENT
    prev = L.qattn_set_kernel(KERNEL_ONE_BLOCK)
    try:
        o0, l0 = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, **kw)
        assert L.qattn_last_kernel() == KERNEL_ONE_BLOCK
        L.qattn_set_kernel(_lib.QATTN_KERNEL_AUTO)
        o1, l1 = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, **kw)
        assert L.qattn_last_kernel() == KERNEL_RESIDENT
        o2, l2 = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, **kw)
    finally:
        L.qattn_set_kernel(prev)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2), "resident kernel is not deterministic"
    assert torch.equal(o0, o1), f"resident kernel differs: max {float((o0.float() - o1.float()).abs().max()):.4g}"
    assert torch.equal(l0, l1)
    if case == "empty_batch":  # no valid key: zero output, LSE -inf
        assert bool((o1[1] == 0).all()) and bool(torch.isneginf(l1[1]).all())
    if case == "padding":
        ref = oracle.qattn_fwd(q8.contiguous().cpu().numpy(), qs.cpu().numpy(), k8.contiguous().cpu().numpy(),
                               ks.cpu().numpy(), v8=untile_v(v8), v_scale=vs.cpu().numpy(), kv_valid=kv_valid,
                               lazy_tau=KERNEL_LAZY_TAU, lsum_rounded=KERNEL_LSUM_ROUNDED, p_linear=KERNEL_P_LINEAR)
        c = cosine(o1.float().cpu().numpy(), ref)
        log(f"  resident padding cos_oracle={c:.6f}")
        assert c >= COS_KERNEL


@pytest.mark.parametrize("case", ["ragged", "padding", "empty_batch", "causal", "causal_odd", "gqa_hnd_thread",
                                  "fp16_warp_gqa", "long", "tiny", "causal_tiny", "one_key_valid", "gqa5_smooth_v",
                                  "split3", "split_causal", "split_thread_gqa_hnd", "split_padding_empty",
                                  "split_causal_offset"])
def test_pingpong_kernel_matches(oracle, case):
    """The ping-pong kernel (two 4-wave groups per workgroup alternating matrix and vector stages) runs the
    same per-element arithmetic and accumulation order as qattn_fwd_kernel, so its output and LSE must be
    identical, bit for bit, on the same quantized operands.  Both kernels are forced through
    qattn_set_kernel whatever the grid size, and qattn_last_kernel confirms which one ran.  Checked on
    ragged lengths (masked tail tiles), key padding per batch (one batch with no valid key at all),
    top-left causal, causal with an odd number of query blocks and more keys than queries, GQA + HND +
    per-thread scales, GQA + per-warp scales + fp16 output, and a key range long enough for the
    steady-state pipeline; also one query over one key, a causal launch with fewer keys than queries, a
    batch whose entries keep 1, 64 and 65 keys (tile boundaries), and GQA with five query heads per key
    head and smoothed V; and KV-split launches (the same split on both kernels: identical partials, one
    combine), including causal, per-thread scales with GQA and HND, and a batch entry without keys whose
    splits are all empty.  The long and some small cases are also checked against the oracle (the split
    ones on the oracle's split schedule)."""
    dev = require_gpu()
    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa

    B, Lq, Lk, Hq, Hkv, layout, causal, kv_valid, gran = {
        "ragged": (2, 1000, 777, 3, 3, "NHD", False, None, "per_block"),
        "padding": (1, 600, 512, 4, 4, "NHD", False, [300], "per_block"),
        "empty_batch": (2, 700, 600, 2, 2, "NHD", False, [600, 0], "per_block"),
        "causal": (1, 1024, 1024, 2, 2, "NHD", True, None, "per_block"),
        "causal_odd": (2, 1100, 1300, 2, 2, "NHD", True, [1300, 900], "per_block"),
        "gqa_hnd_thread": (1, 2000, 1500, 4, 2, "HND", False, None, "per_thread"),
        "fp16_warp_gqa": (1, 900, 1100, 6, 2, "NHD", False, None, "per_warp"),
        "long": (1, 700, 8200, 2, 2, "NHD", False, None, "per_block"),
        "tiny": (1, 1, 1, 2, 2, "NHD", False, None, "per_block"),
        "causal_tiny": (1, 5, 3, 2, 2, "NHD", True, None, "per_block"),
        "one_key_valid": (3, 300, 200, 2, 2, "NHD", False, [1, 64, 65], "per_block"),
        "gqa5_smooth_v": (1, 500, 900, 10, 2, "NHD", False, None, "per_block"),
        "split3": (1, 700, 5000, 2, 2, "NHD", False, None, "per_block"),
        "split_causal": (1, 1100, 1300, 2, 2, "NHD", True, None, "per_block"),
        "split_thread_gqa_hnd": (1, 900, 3000, 4, 2, "HND", False, None, "per_thread"),
        "split_padding_empty": (2, 400, 5000, 2, 2, "NHD", False, [2100, 0], "per_block"),
        "split_causal_offset": (1, 700, 4000, 2, 2, "NHD", True, None, "per_block"),
    }[case]
    ns = {"split3": 3, "split_causal": 2, "split_thread_gqa_hnd": 4, "split_padding_empty": 5,
          "split_causal_offset": 4}.get(case, 1)
    q_offset = 3000 if case == "split_causal_offset" else 0  # a chunk of queries after 3000 earlier keys
    log(f"pingpong vs one-block: {case} B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} layout={layout} causal={causal} "
        f"kv_valid={kv_valid} gran={gran}")
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, seed=4242, k_offset_std=0.5)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    if layout == "HND":
        qd, kd, vd = (t.transpose(1, 2).contiguous() for t in (qd, kd, vd))
    km = sa.k_mean(kd, layout)
    qk_mult = 1.0
    if gran == "per_block":
        q8, qs, k8, ks = sa.per_block_int8(qd, kd, km, sm_scale=128 ** -0.5, tensor_layout=layout)
    else:
        quant = sa.per_thread_int8 if gran == "per_thread" else sa.per_warp_int8
        q8, qs, k8, ks = quant(qd, kd, km, tensor_layout=layout)
        qk_mult = 128 ** -0.5 * LOG2E
    v8, vs, vm = sa.per_channel_fp8(vd, tensor_layout=layout, smooth_v=case == "gqa5_smooth_v")
    out_dtype = torch.float16 if case == "fp16_warp_gqa" else torch.bfloat16
    kw = dict(tensor_layout=layout, out_dtype=out_dtype, is_causal=causal, kv_valid_len=kv_valid,
              return_lse=True, qk_mult=qk_mult, qk_quant_gran=gran, num_splits=ns, v_mean=vm, q_offset=q_offset)
    L = _lib.load()
    prev = L.qattn_set_kernel(KERNEL_ONE_BLOCK)
    try:
        o0, l0 = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, **kw)
        assert L.qattn_last_kernel() == KERNEL_ONE_BLOCK
        L.qattn_set_kernel(KERNEL_PINGPONG)
        o1, l1 = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, **kw)
        assert L.qattn_last_kernel() == KERNEL_PINGPONG
        o2, l2 = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, **kw)
    finally:
        L.qattn_set_kernel(prev)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2), "ping-pong kernel is not deterministic"
    assert torch.equal(o0, o1), f"ping-pong kernel differs: max {float((o0.float() - o1.float()).abs().max()):.4g}"
    assert torch.equal(l0, l1)
    if case == "empty_batch":  # no valid key: zero output, LSE -inf
        assert bool((o1[1] == 0).all()) and bool(torch.isneginf(l1[1]).all())
    if case in ("tiny", "one_key_valid", "gqa5_smooth_v", "causal_tiny", "split3", "split_causal",
                "split_thread_gqa_hnd", "split_padding_empty", "split_causal_offset"):
        nkb = (Lk + 63) // 64
        if layout == "HND":
            o1, q8, k8 = o1.transpose(1, 2), q8.transpose(1, 2), k8.transpose(1, 2)
        ref, ref_lse = oracle.qattn_fwd(q8.contiguous().cpu().numpy(), qs.cpu().numpy(),
                                        k8.contiguous().cpu().numpy(), ks.cpu().numpy(), v8=untile_v(v8),
                                        v_scale=vs.cpu().numpy(), causal=causal, q_offset=q_offset,
                                        kv_valid=kv_valid, want_lse=True,
                                        v_mean=None if vm is None else vm.cpu().numpy(), qk_mult=qk_mult,
                                        q_gran=GRAN_CODE[gran], k_gran=GRAN_CODE[gran],
                                        tiles_per_split=(nkb + ns - 1) // ns if ns > 1 else 0,
                                        lazy_tau=KERNEL_LAZY_TAU, lsum_rounded=KERNEL_LSUM_ROUNDED,
                               p_linear=KERNEL_P_LINEAR)
        og = o1.float().cpu().numpy()
        c = cosine(og, ref)
        lerr = lse_max_err(l1.cpu().numpy(), ref_lse, og.transpose(0, 2, 1, 3))
        log(f"  ping-pong kernel vs quantized oracle: cosine={c:.6f} max_abs={float(np.abs(og - ref).max()):.3g} "
            f"lse_max_abs={lerr:.3g}")
        assert c >= COS_KERNEL and lerr < 2e-2
    if case == "long":
        ref = oracle.qattn_fwd(q8.contiguous().cpu().numpy(), qs.cpu().numpy(), k8.contiguous().cpu().numpy(),
                               ks.cpu().numpy(), v8=untile_v(v8), v_scale=vs.cpu().numpy(),
                               lazy_tau=KERNEL_LAZY_TAU, lsum_rounded=KERNEL_LSUM_ROUNDED,
                               p_linear=KERNEL_P_LINEAR)
        c = cosine(o1.float().cpu().numpy(), ref)
        log(f"  ping-pong kernel vs quantized oracle: cosine={c:.6f}")
        assert c >= COS_KERNEL


@pytest.mark.parametrize("name,call", [("c2", "qattn"), ("c2", "telefuser"), ("c3", "qattn"), ("c4", "qattn"),
                                       ("c5", "qattn")])
def test_full_size_configs(oracle, name, call):
    """BASELINE configs 2-5 at full size through the drop-in's quantize + attention path (the bench's own
    inputs and calls): the Wan2.1-1.3B 480p self attention of the headline number (L = 32760, H = 12, q and
    k after RMSNorm + 3-D RoPE), 14B 720p self attention (L = 75600, H = 40, K mean offset), the 14B text
    cross attention (Lk = 512 with zero-padded, masked keys) and the streaming chunk over a 32760-key
    window (KV split, restated by the oracle).  call="qattn" is the per-block quantizers + qattn_fwd, and
    the benchmark's step (the fused K/V prologue + qattn_fwd_q16, Q quantized inside the attention kernel)
    must give the same bits; call="telefuser" is TeleFuser's own call (attention_impl.py:249-258):
    sageattn_qk_int8_pv_fp8_cuda with per-thread scales and "fp32+fp32" accumulation, checked against the
    oracle on the per-thread operands that the module's quantizers produce for the same inputs.
    Checked on a subset that the CPU finishes in seconds: 192 query rows (the first 128 and the last 64) of
    the first and last head, against float64 truth (cosine >= 0.999) and against the oracle on the very
    quantized operands of the launch (cosine >= 0.99995); the whole output must be finite."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa
    from telefuser_amd.workloads import CONFIGS, make_inputs

    cfg = CONFIGS[name]
    log(f"full size {name} ({call}): B={cfg.B} Lq={cfg.Lq} Lk={cfg.Lk} H={cfg.Hq} pad={cfg.pad_range}")
    q, k, v, kvv = make_inputs(cfg, dev)
    sm = cfg.D ** -0.5
    km = sa.k_mean(k, "NHD")
    if call == "telefuser":
        gran, qk_mult, qpb = 3, sm * LOG2E, 32  # q scales per 128-row block
        o = sa.sageattn_qk_int8_pv_fp8_cuda(q, k, v, tensor_layout="NHD", is_causal=False,
                                            qk_quant_gran="per_thread", sm_scale=sm, pv_accum_dtype="fp32+fp32")
        q8, qs, k8, ks = sa.per_thread_int8(q, k, km, tensor_layout="NHD")
    else:
        gran, qk_mult, qpb = 1, 1.0, 1
        q8, qs, k8, ks = sa.per_block_int8(q, k, km, sm_scale=sm, tensor_layout="NHD")
    v8, vs, _ = sa.per_channel_fp8(v, tensor_layout="NHD", smooth_v=False)
    if call == "qattn":
        o = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, tensor_layout="NHD", out_dtype=q.dtype, kv_valid_len=kvv)
        if sa.q16_supported(cfg.B, cfg.Lq, cfg.Lk, cfg.Hq, cfg.D, "per_block"):
            _, _, k8b, ksb, _, v8b, vsb, _ = sa.sage_quant(q, k, v, tensor_layout="NHD", sm_scale=sm, quantize_q=False)
            o16 = sa.qattn_fwd_q16(q, k8b, ksb, v8b, vsb, tensor_layout="NHD", qk_mult=sm * LOG2E, kv_valid_len=kvv,
                                   qk_quant_gran="per_block")
            torch.cuda.synchronize()
            assert torch.equal(o16, o), f"bench route differs: {float((o16.float() - o.float()).abs().max())}"
            del o16, k8b, v8b
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o.float()).all())
    rows = torch.cat([torch.arange(0, 128), torch.arange(cfg.Lq - 64, cfg.Lq)])
    v8_plain = untile_v(v8)
    from telefuser_amd import _lib
    nkb = (cfg.Lk + 63) // 64
    ns = min(_lib.load().qattn_fwd_ex_num_splits(cfg.B, cfg.Lq, cfg.Lk, cfg.Hq, 0, gran), nkb)
    tps = (nkb + ns - 1) // ns if ns > 1 else 0  # the launch's KV-split schedule, restated on the CPU
    log(f"  kv splits={ns}")
    for h in (0, cfg.Hq - 1):
        og = o[:, rows, h:h + 1].float().cpu().numpy()
        truth = oracle.attn_fp64(bf16_bits(q[:, rows, h:h + 1].cpu()), bf16_bits(k[:, :, h:h + 1].cpu()),
                                 bf16_bits(v[:, :, h:h + 1].cpu()), sm, kv_valid=kvv)
        # the oracle restates quantized rows with their own block's q scales: rows 0..127 are query block 0,
        # the last 64 rows lie inside the last (ragged) block, which is handed over whole
        q8h = q8[:, :, h:h + 1].cpu()
        qsh = qs[:, h:h + 1].cpu().numpy()
        nqb = qsh.shape[-1] // qpb
        kw = dict(v8=np.ascontiguousarray(v8_plain[:, h:h + 1]), v_scale=vs[:, h:h + 1].cpu().numpy(),
                  kv_valid=kvv, lazy_tau=KERNEL_LAZY_TAU, lsum_rounded=KERNEL_LSUM_ROUNDED, p_linear=KERNEL_P_LINEAR,
                  tiles_per_split=tps,
                  qk_mult=qk_mult, q_gran=gran, k_gran=gran)
        k8h, ksh = k8[:, :, h:h + 1].contiguous().cpu().numpy(), ks[:, h:h + 1].cpu().numpy()
        ref_first = oracle.qattn_fwd(q8h[:, :128].contiguous().numpy(), qsh[..., :qpb].copy(), k8h, ksh, **kw)
        last0 = (nqb - 1) * 128  # first row of the last query block
        ref_last = oracle.qattn_fwd(q8h[:, last0:].contiguous().numpy(), qsh[..., (nqb - 1) * qpb:].copy(),
                                    k8h, ksh, **kw)
        ref = np.concatenate([ref_first, ref_last[:, -64:]], axis=1)
        ct, ck = cosine(og, truth), cosine(og, ref)
        log(f"  head {h}: cos_truth={ct:.6f} cos_oracle={ck:.6f} max_abs_truth={float(np.abs(og - truth).max()):.4g} "
            f"max_abs_oracle={float(np.abs(og - ref).max()):.4g}")
        assert ct >= COS_E2E
        assert ck >= COS_KERNEL


@pytest.mark.parametrize("mode", ["fp32_smooth_v", "fp32+fp16", "fp32+fp32_smooth_ignored"])
def test_pv_accum_modes_and_smooth_v(oracle, mode):
    """sageattn_qk_int8_pv_fp8_cuda's pv_accum_dtype / smooth_v semantics (sageattn2.py:1368-1445):
    "fp32" with smooth_v quantizes V - mean and adds the mean back in the epilogue (fuse_v_mean kernel);
    "fp32+fp16" quantizes V with scale_max 2.25 (the reference then sums each tile's P.V in fp16 - this
    kernel sums it in fp32); with "fp32+fp32" smooth_v is ignored with a warning.  Each is checked
    against the oracle on the same quantized operands (the fp16 tile partials restated for "fp32+fp16")
    and against float64 truth."""
    import warnings

    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    B, Lq, Lk, H = 1, 700, 900, 2
    q, k, v = qkv(B, Lq, Lk, H, H, seed=91, k_offset_std=0.5)
    v = (v.float() + 1.5).to(torch.bfloat16)  # a channel offset that smoothing removes
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    pv, smooth = {"fp32_smooth_v": ("fp32", True), "fp32+fp16": ("fp32+fp16", False),
                  "fp32+fp32_smooth_ignored": ("fp32+fp32", True)}[mode]
    log(f"pv_accum {mode}: B={B} Lq={Lq} Lk={Lk} H={H}")
    with warnings.catch_warnings(record=True) as wlist:
        warnings.simplefilter("always")
        o = sa.sageattn_qk_int8_pv_fp8_cuda(qd, kd, vd, tensor_layout="NHD", qk_quant_gran="per_thread",
                                            pv_accum_dtype=pv, smooth_v=smooth)
    torch.cuda.synchronize()
    assert any("smooth_v will be ignored" in str(w.message) for w in wlist) == (mode == "fp32+fp32_smooth_ignored")
    og = o.float().cpu().numpy()
    # the same operands, quantized on the GPU by the module's own quantizers
    km = sa.k_mean(kd, "NHD")
    q8, qs, k8, ks = sa.per_thread_int8(qd, kd, km, tensor_layout="NHD")
    use_smooth = mode == "fp32_smooth_v"
    v8, vs, vm = sa.per_channel_fp8(vd, tensor_layout="NHD", scale_max=2.25 if pv == "fp32+fp16" else 448.0,
                                    smooth_v=use_smooth)
    args = (q8.cpu().numpy(), qs.cpu().numpy(), k8.cpu().numpy(), ks.cpu().numpy())
    kw = dict(v8=untile_v(v8), v_scale=vs.cpu().numpy(), qk_mult=128 ** -0.5 * LOG2E, q_gran=3, k_gran=3,
              v_mean=None if vm is None else vm.cpu().numpy())
    ref_k = oracle.qattn_fwd(*args, **kw, lazy_tau=KERNEL_LAZY_TAU, lsum_rounded=KERNEL_LSUM_ROUNDED,
                               p_linear=KERNEL_P_LINEAR)
    ref_r = oracle.qattn_fwd(*args, **kw, pv_f16_tile=pv == "fp32+fp16")
    truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(k), bf16_bits(v), 128 ** -0.5)
    ck, cr, ct = cosine(og, ref_k), cosine(og, ref_r), cosine(og, truth)
    log(f"  cos kernel-schedule oracle={ck:.6f} reference math={cr:.6f} truth={ct:.6f} "
        f"max_abs_truth={float(np.abs(og - truth).max()):.4g}")
    assert ck >= COS_KERNEL
    assert cr >= COS_E2E
    assert ct >= COS_E2E


Q16_CASES = {
    # name: (B, Lq, Lk, Hq, Hkv, layout, dtype, gran, kv_valid, smooth_v, causal); the first nine run the
    # resident kernel (at most 512 keys), the others the ping-pong kernel (unsplit, KV split, causal)
    "thread_c4_like": (1, 1000, 512, 4, 4, "NHD", torch.bfloat16, "per_thread", [388], False, False),
    "warp_ragged_gqa": (2, 333, 300, 4, 2, "NHD", torch.bfloat16, "per_warp", None, False, False),
    "thread_hnd_fp16": (1, 517, 130, 3, 3, "HND", torch.float16, "per_thread", None, False, False),
    "thread_smooth_v_short_q": (2, 40, 64, 2, 1, "NHD", torch.bfloat16, "per_thread", [64, 17], True, False),
    "warp_fp16_keys_512": (1, 777, 512, 2, 2, "NHD", torch.float16, "per_warp", None, True, False),
    # per block on the resident kernel: chunks of whole 128-row blocks (12 rows of 32 in three chunks; a ragged
    # last block; 200 heads in one chunk each, so three rounds per wave with a partial last group)
    "block_res_chunks": (1, 1000, 512, 4, 4, "NHD", torch.bfloat16, "per_block", [388], False, False),
    "block_res_hnd_fp16": (2, 333, 300, 4, 2, "HND", torch.float16, "per_block", [300, 17], True, False),
    "block_res_rounds_gqa": (5, 900, 200, 40, 8, "NHD", torch.bfloat16, "per_block", None, False, False),
    "block_res_tiny": (1, 20, 100, 2, 1, "NHD", torch.bfloat16, "per_block", [37], False, False),
    "pp_thread_unsplit": (1, 4680, 6000, 12, 12, "NHD", torch.bfloat16, "per_thread", None, False, False),
    "pp_warp_split_gqa": (1, 2000, 20000, 8, 4, "NHD", torch.bfloat16, "per_warp", [19000], False, False),
    "pp_thread_causal_fp16": (2, 1500, 3000, 8, 8, "HND", torch.float16, "per_thread", None, False, True),
    "pp_block_unsplit": (1, 4680, 6000, 12, 12, "NHD", torch.bfloat16, "per_block", None, False, False),
    "pp_block_split_kv_valid": (1, 2000, 20000, 8, 4, "NHD", torch.bfloat16, "per_block", [19000], True, False),
    "pp_block_causal_fp16": (2, 1500, 3000, 8, 8, "HND", torch.float16, "per_block", None, False, True),
}


@pytest.mark.parametrize("gran", ["per_block", "per_warp", "per_thread"])
def test_fwd_q16_causal_query_offset(gran):
    """A streaming chunk through qattn_fwd_q16: 1536 causal queries placed after 2560 earlier keys (q_offset),
    bit-identical to the quantize-then-attend sequence (48 query-block pairs: the automatic rule splits the
    key range of the ping-pong launch)."""
    dev = require_gpu()
    from telefuser_amd import _lib
    from telefuser_amd import sageattn2 as sa

    B, Lq, Lk, Hq, Hkv = 1, 1536, 4096, 8, 4
    log(f"fwd_q16 causal q_offset: {gran} B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} q_offset={Lk - Lq}")
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, seed=57, k_offset_std=0.5)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    km = sa.k_mean(kd, "NHD")
    qk_mult = 128 ** -0.5 * LOG2E
    if gran == "per_block":
        q8, qs, k8, ks = sa.per_block_int8(qd, kd, km, sm_scale=128 ** -0.5, tensor_layout="NHD")
    else:
        quant = sa.per_thread_int8 if gran == "per_thread" else sa.per_warp_int8
        q8, qs, k8, ks = quant(qd, kd, km, tensor_layout="NHD")
    v8, vs, _ = sa.per_channel_fp8(vd, tensor_layout="NHD")
    assert sa.q16_supported(B, Lq, Lk, Hq, 128, gran, True)
    L = _lib.load()
    log(f"  automatic splits: {L.qattn_fwd_ex_num_splits(B, Lq, Lk, Hq, _lib.QATTN_V_FP8, GRAN_CODE[gran])}")
    kw = dict(tensor_layout="NHD", is_causal=True, q_offset=Lk - Lq, return_lse=True, qk_quant_gran=gran)
    o_ref, l_ref = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, out_dtype=q.dtype,
                                qk_mult=1.0 if gran == "per_block" else qk_mult, **kw)
    o, l = sa.qattn_fwd_q16(qd, k8, ks, v8, vs, qk_mult=qk_mult, **kw)
    torch.cuda.synchronize()
    assert L.qattn_last_kernel() == _lib.QATTN_KERNEL_PINGPONG
    assert torch.equal(o, o_ref), f"max diff {float((o.float() - o_ref.float()).abs().max())}"
    assert torch.equal(l, l_ref)


@pytest.mark.parametrize("case", sorted(Q16_CASES))
def test_fwd_q16_matches_quantize_then_attend(oracle, case):
    """qattn_fwd_q16 quantizes Q inside the attention kernel: its output and LSE must be bit-identical to
    per_thread_int8 / per_warp_int8 / per_block_int8 followed by qattn_fwd on the same K / V, and the drop-in
    (which takes this route where qattn_fwd_q16 covers the launch) must give the same bits as well."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    B, Lq, Lk, Hq, Hkv, layout, dt, gran, kv_valid, smooth_v, causal = Q16_CASES[case]
    log(f"fwd_q16 {case}: B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} {layout} {dt} {gran} kv_valid={kv_valid} "
        f"causal={causal}")
    assert sa.q16_supported(B, Lq, Lk, Hq, 128, gran, causal)
    q, k, v = qkv(B, Lq, Lk, Hq, Hkv, seed=53, k_offset_std=0.5, dtype=dt)
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    if layout == "HND":
        qd, kd, vd = (t.transpose(1, 2).contiguous() for t in (qd, kd, vd))
    km = sa.k_mean(kd, layout)
    qk_mult = 128 ** -0.5 * LOG2E
    if gran == "per_block":  # sm_scale * log2(e) folded into Q's scales
        q8, qs, k8, ks = sa.per_block_int8(qd, kd, km, sm_scale=128 ** -0.5, tensor_layout=layout)
    else:
        quant = sa.per_thread_int8 if gran == "per_thread" else sa.per_warp_int8
        q8, qs, k8, ks = quant(qd, kd, km, tensor_layout=layout)
    v8, vs, vm = sa.per_channel_fp8(vd, tensor_layout=layout, smooth_v=smooth_v)
    o_ref, l_ref = sa.qattn_fwd(q8, qs, k8, ks, v8, vs, tensor_layout=layout, out_dtype=dt,
                                qk_mult=1.0 if gran == "per_block" else qk_mult, is_causal=causal,
                                kv_valid_len=kv_valid, return_lse=True, qk_quant_gran=gran, v_mean=vm)
    o, l = sa.qattn_fwd_q16(qd, k8, ks, v8, vs, tensor_layout=layout, qk_mult=qk_mult, is_causal=causal,
                            kv_valid_len=kv_valid, return_lse=True, qk_quant_gran=gran, v_mean=vm)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref), f"max diff {float((o.float() - o_ref.float()).abs().max())}"
    assert torch.equal(l, l_ref)
    # the drop-in on the same inputs: identical to its quantize-then-attend steps
    kw = dict(tensor_layout=layout, qk_quant_gran=gran, pv_accum_dtype="fp32" if smooth_v else "fp32+fp32",
              smooth_v=smooth_v, kv_valid_len=kv_valid, return_lse=True, is_causal=causal)
    od, ld = sa.sageattn_qk_int8_pv_fp8_cuda(qd, kd, vd, **kw)
    torch.cuda.synchronize()
    assert torch.equal(od, o)
    # and within the north star's bound of the reference's quantized math (its own schedule, e4m3(exp2) P) on
    # the same int8 / e4m3 operands: batch entry 0, the first 256 rows of heads 0 and 1 and their KV heads
    # (float64 attention on the half inputs is printed: with smoothed V over 19000 keys of flat random
    # attention the reference's math itself lands at 0.99897 from it, so it is not a gate here)
    if layout == "HND":
        od, q8, k8 = od.transpose(1, 2), q8.transpose(1, 2), k8.transpose(1, 2)
    rows, nkv = slice(0, min(Lq, 256)), max(1, 2 * Hkv // Hq)
    q_per = {"per_block": 1, "per_warp": 4, "per_thread": 32}[gran]
    kvv0 = None if kv_valid is None else kv_valid[:1]
    ref = oracle.qattn_fwd(q8[:1, rows, :2].contiguous().cpu().numpy(), qs[:1, :2, :2 * q_per].cpu().numpy(),
                           k8[:1, :, :nkv].contiguous().cpu().numpy(), ks[:1, :nkv].cpu().numpy(),
                           v8=untile_v(v8[:1, :nkv]), v_scale=vs[:1, :nkv].cpu().numpy(), causal=causal,
                           kv_valid=kvv0, q_gran=GRAN_CODE[gran], k_gran=GRAN_CODE[gran],
                           qk_mult=1.0 if gran == "per_block" else qk_mult,
                           v_mean=None if vm is None else vm[:1, :nkv].cpu().numpy())
    got = od[:1, rows, :2].float().cpu().numpy()
    bits = (lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)) if dt == torch.float16 else bf16_bits
    truth = oracle.attn_fp64(bits(q[:1, rows, :2]), bits(k[:1, :, :nkv]), bits(v[:1, :, :nkv]), 128 ** -0.5,
                             kv_valid=kvv0, is_fp16=dt == torch.float16, causal=causal)
    log(f"  vs reference-schedule quantized math: cosine={cosine(got, ref):.6f}; vs float64: {cosine(got, truth):.6f}")
    assert cosine(got, ref) >= COS_E2E


@pytest.mark.parametrize("gran,lk", [("per_block", 3000), ("per_thread", 3000), ("per_block", 300),
                                     ("per_thread", 300)])
def test_dropin_strided_views_of_packed_qkv(gran, lk):
    """q, k and v as views of one packed [B, L, 3, H, D] projection output (row strides 3 H D, last dim
    contiguous), through the drop-in, whose Q goes straight into the attention kernel (qattn_fwd_q16 on the
    ping-pong kernel for 3000 keys, on the resident kernel for 300): the same bits as contiguous copies."""
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    B, L, H, D = 1, lk, 4, 128
    log(f"strided packed qkv: {gran} B={B} L={L} H={H}")
    g = torch.Generator().manual_seed(61)
    qkv_packed = torch.randn(B, L, 3, H, D, generator=g).to(torch.bfloat16).to(dev)
    q, k, v = qkv_packed[:, :, 0], qkv_packed[:, :, 1], qkv_packed[:, :, 2]
    assert not q.is_contiguous() and q.stride(1) == 3 * H * D
    assert sa.q16_supported(B, L, L, H, D, gran, False)
    kw = dict(tensor_layout="NHD", qk_quant_gran=gran, pv_accum_dtype="fp32+fp32", return_lse=True)
    o, lse = sa.sageattn_qk_int8_pv_fp8_cuda(q, k, v, **kw)
    oc, lsec = sa.sageattn_qk_int8_pv_fp8_cuda(q.contiguous(), k.contiguous(), v.contiguous(), **kw)
    torch.cuda.synchronize()
    assert torch.equal(o, oc), f"max diff {float((o.float() - oc.float()).abs().max())}"
    assert torch.equal(lse, lsec)
