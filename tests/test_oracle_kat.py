"""Pins the CPU oracle before anything is checked against it.

The reference ships no golden vectors for this path (its only test compares against fp attention
at rtol/atol 0.1-0.15, tf-kernel/tests/test_sageattn2.py:127-244), so every oracle function is
pinned here by closed-form known answers, by torch's own casts, by an independent float32 numpy
restatement, by brute-force float64 attention and by softmax invariances.  Each check is chosen so
that a plausible slip (RNE vs half-away rounding, a missing amax floor, km applied in the wrong
precision, a dropped sm_scale, a transposed operand, a wrong tile max) fails at least one of them.
"""

import math

import numpy as np
import pytest
import torch

from tests.inputs import bf16_bits, cosine, qkv

LOG2E = 1.44269504


def _bits(vals, shape):
    return bf16_bits(torch.tensor(vals, dtype=torch.float32).reshape(shape))


# ------------------------------------------------------------------------------------------------
# scalar conversions
# ------------------------------------------------------------------------------------------------

def _float_sweep():
    """Every fp32 whose low 16 bits are one of a set of tie / near-tie patterns, plus randoms."""
    hi = np.arange(0, 1 << 16, dtype=np.uint32)
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1234], np.uint32)
    u = (hi[:, None] << 16 | lows[None, :]).ravel()
    f = u.view(np.float32)
    f = f[np.isfinite(f)]
    rng = np.random.default_rng(1)
    return np.concatenate([f, rng.standard_normal(1 << 18).astype(np.float32) * 50])


def test_e4m3_matches_torch_cast_in_range(oracle):
    x = _float_sweep()
    x = x[np.abs(x) < 448.0]
    got = oracle.cvt_array(x, "e4m3")
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)


def test_e4m3_known_answers_and_satfinite(oracle):
    cases = {
        0.0: 0x00, 448.0: 0x7E, 447.99: 0x7E, 460.0: 0x7E, 1e9: 0x7E, float("inf"): 0x7E, -1e9: 0xFE,
        -448.0: 0xFE, 1.0: 0x38, 1.0625: 0x38, 1.1875: 0x3A, 2 ** -9: 0x01, 2 ** -10: 0x00,
        3 * 2 ** -10: 0x02, 2 ** -6: 0x08, 240.0: 0x77, 2 ** 8.807: 0x7E,
    }
    for x, b in cases.items():
        assert oracle.lib().oq_f32_to_e4m3(x) == b, (x, hex(b))
    # decode round trip of every finite code
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    vals = oracle.e4m3_to_f32(codes)
    assert np.array_equal(oracle.cvt_array(vals, "e4m3")[codes != 0x80], codes[codes != 0x80])
    assert vals.max() == 448.0 and vals[vals > 0].min() == 2 ** -9


def test_bf16_rne_matches_torch(oracle):
    x = _float_sweep()
    got = oracle.cvt_array(x, "bf16")
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_rne_matches_torch(oracle):
    x = _float_sweep()
    got = oracle.cvt_array(x, "f16")
    want = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    finite = np.isfinite(torch.from_numpy(x).to(torch.float16).numpy())
    assert np.array_equal(got[finite], want[finite])


def test_s8_rounding_kats(oracle):
    x = np.array([2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 126.5, 127.4, 127.6, 200, -129, -127.5, 1.49999],
                 np.float32)
    rne = oracle.cvt_array(x, "s8_rne")
    away = oracle.cvt_array(x, "s8_half_away")
    assert rne.tolist() == [2, -2, 4, -4, 0, 0, 126, 127, 127, 127, -128, -128, 1]
    assert away.tolist() == [3, -3, 4, -4, 1, -1, 127, 127, 127, 127, -128, -128, 1]


# ------------------------------------------------------------------------------------------------
# per-block INT8 quantizer (CUDA QuantInt8Kernel semantics)
# ------------------------------------------------------------------------------------------------

def test_quant_all_zero_block_uses_amax_floor(oracle):
    x = np.zeros((1, 64, 1, 128), np.uint16)
    q, s = oracle.quant_per_block_int8(x, blk=64)
    assert np.all(q == 0)
    assert s[0, 0, 0] == np.float32(np.float32(1e-7) / np.float32(127.0))


def test_quant_ties_are_round_half_even(oracle):
    vals = np.zeros((64, 128), np.float32)
    vals[0, 0] = 127.0  # amax 127 -> inv = 1 exactly
    vals[0, 1:9] = [2.5, -2.5, 3.5, -3.5, 0.5, -0.5, -127.0, 1.5]
    q, s = oracle.quant_per_block_int8(_bits(vals, (1, 64, 1, 128)), blk=64)
    assert s[0, 0, 0] == np.float32(1.0)
    assert q[0, 0, 0, :9].tolist() == [127, 2, -2, 4, -4, 0, 0, -127, 2]


def test_quant_triton_variant_ties_away_and_no_floor(oracle):
    vals = np.zeros((64, 128), np.float32)
    vals[0, 0] = 127.0
    vals[0, 1:5] = [2.5, -2.5, 0.5, -0.5]
    q, s = oracle.quant_per_block_int8(_bits(vals, (1, 64, 1, 128)), blk=64, variant="triton")
    assert q[0, 0, 0, :5].tolist() == [127, 3, -3, 1, -1]
    z, sz = oracle.quant_per_block_int8(np.zeros((1, 64, 1, 128), np.uint16), blk=64, variant="triton")
    assert sz[0, 0, 0] == 0.0 and np.all(z == 0)


def test_quant_ragged_tail_rows_excluded(oracle):
    L = 130
    vals = np.ones((L, 128), np.float32)
    vals[:128] *= 0.25
    vals[128:] = 4.0
    vals[129, 3] = -8.0
    q, s = oracle.quant_per_block_int8(_bits(vals, (1, L, 1, 128)), blk=128)
    assert s.shape == (1, 1, 2)
    assert s[0, 0, 0] == np.float32(0.25) / np.float32(127)
    assert s[0, 0, 1] == np.float32(8.0) / np.float32(127)
    assert q[0, 129, 0, 3] == -127 and q[0, 128, 0, 0] == 64  # 4*127/8 = 63.5 -> 64 (RNE, even)


def test_quant_km_subtracted_in_fp32(oracle):
    # x - km is not bf16-representable: the CUDA path keeps the fp32 difference, Triton rounds it
    x = np.full((64, 128), 1.0078125, np.float32)
    km = np.full((1, 1, 128), 2 ** -9, np.float32)
    xb, kb = _bits(x, (1, 64, 1, 128)), _bits(km, (1, 1, 128))
    _, s_cuda = oracle.quant_per_block_int8(xb, km_bits=kb, blk=64)
    _, s_tri = oracle.quant_per_block_int8(xb, km_bits=kb, blk=64, variant="triton")
    assert s_cuda[0, 0, 0] == np.float32(1.005859375) / np.float32(127)
    assert s_tri[0, 0, 0] == np.float32(1.0078125) / np.float32(127)


def test_quant_sm_scale_is_fp32_of_the_python_double(oracle):
    D = 128
    sm = D ** -0.5 * LOG2E
    vals = np.zeros((128, D), np.float32)
    vals[0, 0] = 3.0
    vals[5, 7] = 1.0
    q, s = oracle.quant_per_block_int8(_bits(vals, (1, 128, 1, D)), sm_scale=sm, blk=128)
    f = np.float32(sm)
    amax = np.float32(3.0) * f
    assert s[0, 0, 0] == amax / np.float32(127)
    inv = np.float32(127) / amax
    assert q[0, 5, 0, 7] == np.rint(np.float32(np.float32(1.0) * f) * inv)  # 42.333 -> 42


def _numpy_quant(xf, kmf, sm, blk):
    """Independent vectorised float32 restatement (numpy's float32 ops are IEEE-rounded)."""
    B, L, H, D = xf.shape
    n = (L + blk - 1) // blk
    x = xf.astype(np.float32)
    if kmf is not None:
        x = (x - kmf[:, None, :, :].astype(np.float32)).astype(np.float32)
    if sm is not None:
        x = (x * np.float32(sm)).astype(np.float32)
    pad = np.zeros((B, n * blk, H, D), np.float32)
    pad[:, :L] = x
    blocks = pad.reshape(B, n, blk, H, D)
    amax = np.maximum(np.abs(blocks).max(axis=(2, 4)), np.float32(1e-7)).astype(np.float32)  # [B, n, H]
    scale = (amax / np.float32(127)).astype(np.float32)
    inv = (np.float32(127) / amax).astype(np.float32)
    qv = np.clip(np.rint((blocks * inv[:, :, None, :, None]).astype(np.float32)), -128, 127).astype(np.int8)
    return qv.reshape(B, n * blk, H, D)[:, :L], scale.transpose(0, 2, 1)


@pytest.mark.parametrize("L,blk,with_km,with_sm", [(1000, 128, False, True), (777, 64, True, False),
                                                   (64, 64, True, False), (300, 128, False, False)])
def test_quant_random_matches_numpy_restatement(oracle, L, blk, with_km, with_sm):
    q, k, _ = qkv(2, L, L, 3, 3, seed=7, k_offset_std=0.5)
    x = k if with_km else q
    xb = bf16_bits(x)
    xf = oracle.bf16_bits_to_f32(xb)
    kmb = oracle.k_mean_bits(xb) if with_km else None
    kmf = oracle.bf16_bits_to_f32(kmb) if with_km else None
    sm = 128 ** -0.5 * LOG2E if with_sm else None
    got_q, got_s = oracle.quant_per_block_int8(xb, km_bits=kmb, sm_scale=sm, blk=blk)
    want_q, want_s = _numpy_quant(xf, kmf, sm, blk)
    assert np.array_equal(got_s, want_s)
    assert np.array_equal(got_q, want_q)


def test_quant_hnd_layout_equals_nhd(oracle):
    q, _, _ = qkv(1, 200, 200, 2, 2, seed=3)
    nhd = bf16_bits(q)
    hnd = np.ascontiguousarray(nhd.transpose(0, 2, 1, 3))
    a, sa = oracle.quant_per_block_int8(nhd, blk=64, layout="NHD")
    b, sb = oracle.quant_per_block_int8(hnd, blk=64, layout="HND")
    assert np.array_equal(sa, sb)
    assert np.array_equal(a, b.transpose(0, 2, 1, 3))


# ------------------------------------------------------------------------------------------------
# per-channel FP8 V quantizer
# ------------------------------------------------------------------------------------------------

def test_v_fp8_known_answers(oracle):
    v = np.zeros((70, 128), np.float32)
    v[:, 0] = 1.0
    v[3, 0] = 2.0
    v[:, 1] = -0.5
    v[:, 2] = np.linspace(-3, 1, 70)
    v8, vs = oracle.per_channel_fp8(_bits(v, (1, 70, 1, 128)))
    assert v8.shape == (1, 1, 128, 128)
    assert vs[0, 0, 0] == np.float32(2.0) / np.float32(448)
    assert v8[0, 0, 0, 3] == 0x7E and v8[0, 0, 0, 0] == oracle.lib().oq_f32_to_e4m3(224.0)
    assert v8[0, 0, 1, 0] == 0xFE  # -0.5 is the channel's amax -> -448
    assert np.all(v8[0, 0, :, 70:] == 0)  # key slots past L are zero in every channel
    assert np.all(v8[0, 0, 5, :70] == 0x7F)
    assert vs[0, 0, 5] == 0.0  # all-zero channel: scale 0, recp = inf, codes NaN (as the reference)


def test_v_fp8_smooth_known_answers(oracle):
    """sub_mean form of MeanScaleKernel (fused.cu:362-445): mean over the tokens padded with zeros to a
    multiple of 16, amax from max / min about that mean (pad zeros included), v8 = e4m3((v - mean) * recp)."""
    v = np.zeros((70, 128), np.float32)
    v[:, 0] = 2.0             # constant channel, 70 tokens (pad to 80): mean = 1.75, amax = |0 - 1.75|
    v[:, 1] = np.linspace(-3, 1, 70)
    v8, vs, mean = oracle.per_channel_fp8(_bits(v, (1, 70, 1, 128)), smooth=True)
    assert mean[0, 0, 0] == np.float32(2.0 * 70 / 80)
    assert vs[0, 0, 0] == np.float32(1.75) / np.float32(448)
    # (2 - 1.75) * 448 / 1.75 = 64 exactly
    assert np.all(v8[0, 0, 0, :70] == oracle.lib().oq_f32_to_e4m3(64.0))
    assert np.all(v8[0, 0, :, 70:] == 0)
    col = oracle.bf16_bits_to_f32(_bits(v, (1, 70, 1, 128)))[0, :, 0, 1]  # the bf16 values of channel 1
    m1 = np.float32(col.astype(np.float64).sum() / 80)
    assert abs(mean[0, 0, 1] - m1) <= 1e-6
    amax1 = max(abs(np.float32(col.max()) - mean[0, 0, 1]), abs(np.float32(col.min()) - mean[0, 0, 1]))
    assert vs[0, 0, 1] == np.float32(amax1) / np.float32(448)
    # 64 tokens (a multiple of 16): no pad zeros join the max / min
    w = np.full((64, 128), 3.0, np.float32)
    w[0] = 1.0
    _, vs2, mean2 = oracle.per_channel_fp8(_bits(w, (1, 64, 1, 128)), smooth=True)
    assert mean2[0, 0, 0] == np.float32((63 * 3.0 + 1.0) / 64)
    assert vs2[0, 0, 0] == np.float32(abs(1.0 - mean2[0, 0, 0])) / np.float32(448)
    # the mean is taken from mean_in when given (the GPU's reduction order is an input of the bit-exact step)
    _, _, mean3 = oracle.per_channel_fp8(_bits(w, (1, 64, 1, 128)), smooth=True, mean_in=np.full((1, 1, 128), 0.5))
    assert np.all(mean3 == np.float32(0.5))


def test_v_fp8_smooth_matches_numpy_restatement(oracle):
    for L in (96, 333):
        _, _, v = qkv(1, L, L, 2, 2, seed=21)
        vb = bf16_bits(v)
        v8, vs, mean = oracle.per_channel_fp8(vb, smooth=True, scale_max=2.25)
        x = oracle.bf16_bits_to_f32(vb).transpose(0, 2, 3, 1).astype(np.float32)  # B H D L
        l16 = (L + 15) // 16 * 16
        mx, mn = x.max(-1), x.min(-1)
        if l16 != L:
            mx, mn = np.maximum(mx, 0), np.minimum(mn, 0)
        amax = np.maximum(np.abs(mx - mean), np.abs(mn - mean)).astype(np.float32)
        assert np.array_equal(vs, amax / np.float32(2.25))
        recp = np.float32(2.25) / amax
        want = oracle.cvt_array(((x - mean[..., None]).astype(np.float32) * recp[..., None]).astype(np.float32), "e4m3")
        assert np.array_equal(v8[..., :L], want)


def test_v_fp8_random_matches_torch_cast(oracle):
    _, _, v = qkv(2, 333, 333, 3, 3, seed=11)
    vb = bf16_bits(v)
    v8, vs = oracle.per_channel_fp8(vb)
    vf = oracle.bf16_bits_to_f32(vb).transpose(0, 2, 3, 1)  # B H D L
    amax = np.abs(vf).max(axis=-1).astype(np.float32)
    assert np.array_equal(vs, (amax / np.float32(448)).astype(np.float32))
    recp = (np.float32(448) / amax).astype(np.float32)
    y = (vf * recp[..., None]).astype(np.float32)
    want = torch.from_numpy(np.clip(y, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(v8[..., :333], want)


# ------------------------------------------------------------------------------------------------
# attention
# ------------------------------------------------------------------------------------------------

def _numpy_attn(qf, kf, vf, scale, mask=None):
    s = np.einsum("bqhd,bkhd->bhqk", qf.astype(np.float64), kf.astype(np.float64)) * scale
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhqk,bkhd->bqhd", p, vf.astype(np.float64))


def test_fp64_truth_matches_numpy(oracle):
    q, k, v = qkv(1, 70, 90, 2, 2, seed=5)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    got = oracle.attn_fp64(qb, kb, vb, 128 ** -0.5)
    f = oracle.bf16_bits_to_f32
    want = _numpy_attn(f(qb), f(kb), f(vb), 128 ** -0.5)
    assert np.abs(got - want).max() < 1e-6
    # causal (top-left) and key padding
    got_c = oracle.attn_fp64(qb, kb, vb, 128 ** -0.5, causal=True, kv_valid=[60])
    qi, ki = np.arange(70)[:, None], np.arange(90)[None, :]
    mask = (ki <= qi) & (ki < 60)
    want_c = _numpy_attn(f(qb), f(kb), f(vb), 128 ** -0.5, mask[None, None])
    assert np.abs(got_c - want_c).max() < 1e-6


def _pipeline(oracle, q, k, v, smooth=True, pv_mode=0, blkk=64, **kw):
    D = q.shape[-1]
    sm = D ** -0.5
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    kmb = oracle.k_mean_bits(kb) if smooth else None
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=sm * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, km_bits=kmb, blk=blkk)
    if pv_mode == 0:
        v8, vs = oracle.per_channel_fp8(vb, pad=blkk)
        return oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, blkk=blkk, **kw)
    return oracle.qattn_fwd(q8, qs, k8, ks, vh_bits=vb, pv_mode=1, blkk=blkk, **kw)


def test_quantized_pipeline_close_to_truth_c1(oracle):
    # B=1, H=2, L=1024, D=128, k offset N(0, 0.5)
    q, k, v = qkv(1, 1024, 1024, 2, 2, seed=20250101, k_offset_std=0.5)
    truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(k), bf16_bits(v), 128 ** -0.5)
    o8 = _pipeline(oracle, q, k, v, pv_mode=0)
    o16 = _pipeline(oracle, q, k, v, pv_mode=1)
    assert cosine(o8, truth) >= 0.999
    assert cosine(o16, truth) >= 0.999
    assert cosine(o16, truth) > cosine(o8, truth)  # fp8 P/V rounding costs accuracy


def test_dequantized_two_pass_agrees_with_tile_order(oracle):
    """pv_mode 1 differs from exact softmax on the dequantized int8 logits only by bf16 P rounding."""
    q, k, v = qkv(1, 200, 333, 2, 2, seed=9, k_offset_std=1.0)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    sm = 128 ** -0.5
    kmb = oracle.k_mean_bits(kb)
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=sm * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, km_bits=kmb, blk=64)
    got = oracle.qattn_fwd(q8, qs, k8, ks, vh_bits=vb, pv_mode=1)
    qd = q8.astype(np.float64) * np.repeat(qs.transpose(0, 2, 1), 128, axis=1)[:, :200, :, None]
    kd = k8.astype(np.float64) * np.repeat(ks.transpose(0, 2, 1), 64, axis=1)[:, :333, :, None]
    want = _numpy_attn(qd, kd, oracle.bf16_bits_to_f32(vb), math.log(2))  # exp2(s) == exp(s ln2)
    assert cosine(got, want) > 0.99999
    assert np.abs(got - want).max() < 2e-2


def test_smoothing_invariance(oracle):
    """Adding a constant vector to every key leaves softmax unchanged; with K smoothing the
    quantized pipeline output is (nearly) unchanged too, without it accuracy collapses."""
    q, k, v = qkv(1, 256, 512, 1, 1, seed=13)
    shift = torch.randn((1, 1, 1, 128), generator=torch.Generator().manual_seed(2)) * 8.0
    k2 = (k.float() + shift).to(torch.bfloat16)
    truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(k2), bf16_bits(v), 128 ** -0.5)
    smooth = _pipeline(oracle, q, k2, v, smooth=True)
    raw = _pipeline(oracle, q, k2, v, smooth=False)
    assert cosine(smooth, truth) >= 0.999
    assert cosine(smooth, truth) > cosine(raw, truth)


def test_uniform_v_and_single_key(oracle):
    q, k, v = qkv(1, 128, 300, 1, 1, seed=17)
    row = torch.linspace(-2, 2, 128).to(torch.bfloat16)
    vu = row.expand(1, 300, 1, 128).contiguous()
    o = _pipeline(oracle, q, k, vu)
    assert np.abs(o - row.float().numpy()).max() < 0.05 * 2  # fp8 P sum vs fp32 d: ~1% relative
    o1 = _pipeline(oracle, q, k[:, :1], v[:, :1])
    v0 = v[0, 0, 0].float().numpy()
    # single key: p = 2^8.807 -> 448, O = 448/2^8.807 * fp8(V0) * v_scale
    assert np.abs(o1[0, :, 0] - v0[None]).max() <= np.abs(v0).max() * (2 ** -4) + 1e-6


def test_masks_in_quantized_oracle(oracle):
    q, k, v = qkv(1, 192, 192, 2, 2, seed=19)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    truth = oracle.attn_fp64(qb, kb, vb, 128 ** -0.5, causal=True)
    o = _pipeline(oracle, q, k, v, causal=True)
    assert cosine(o, truth) >= 0.999
    truth_p = oracle.attn_fp64(qb, kb, vb, 128 ** -0.5, kv_valid=[100])
    o_p = _pipeline(oracle, q, k, v, kv_valid=[100])
    assert cosine(o_p, truth_p) >= 0.999
    # on the same quantized tensors, the padding mask equals truncating K/V to the valid keys
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=128 ** -0.5 * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, blk=64)
    v8, vs = oracle.per_channel_fp8(vb)
    masked = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, kv_valid=[100])
    trunc = oracle.qattn_fwd(q8, qs, k8[:, :100], ks[:, :, :2], np.ascontiguousarray(v8[..., :128]), vs)
    assert np.array_equal(masked, trunc)


def test_gqa_heads_map_to_kv_groups(oracle):
    q, k, v = qkv(1, 128, 128, 4, 2, seed=23)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    truth = oracle.attn_fp64(qb, kb, vb, 128 ** -0.5)
    o = _pipeline(oracle, q, k, v)
    assert cosine(o, truth) >= 0.999
    # head 3 must use kv head 1: swapping kv heads breaks it
    kb2 = kb[:, :, ::-1].copy()
    assert cosine(oracle.attn_fp64(qb, kb2, vb, 128 ** -0.5), truth) < 0.9


def test_lse_matches_logsumexp(oracle):
    q, k, v = qkv(1, 128, 256, 1, 1, seed=29)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=128 ** -0.5 * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, blk=64)
    v8, vs = oracle.per_channel_fp8(vb)
    _, lse2 = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, want_lse=True)
    qd = q8[0, :, 0].astype(np.float64) * qs[0, 0, 0]
    kd = k8[0, :, 0].astype(np.float64) * np.repeat(ks[0, 0], 64)[:, None]
    s = qd @ kd.T  # log2 domain
    want = np.log2(np.exp2(s - s.max(1, keepdims=True)).sum(1)) + s.max(1)
    assert np.abs(lse2[0, 0] - want).max() < 1e-4


def test_split_schedule_restatement(oracle):
    """One split covering every tile is the unsplit schedule bit for bit; real splits only change
    the fp8 rounding of P (each split has its own running max)."""
    q, k, v = qkv(1, 128, 1000, 1, 1, seed=31)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=128 ** -0.5 * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, blk=64)
    v8, vs = oracle.per_channel_fp8(vb)
    base = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs)
    assert np.array_equal(base, oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, tiles_per_split=16))
    split = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, tiles_per_split=3)
    assert 0.999 < cosine(split, base) < 1.0
    truth = oracle.attn_fp64(qb, kb, vb, 128 ** -0.5)
    assert cosine(split, truth) >= 0.999


def test_lazy_running_max_schedule(oracle):
    """The lazy running-max rule (device kernel schedule) only changes which fp8 rounding P gets:
    tau = 0 with the offset unchanged is the reference rule exactly; tau = 1 and tau = 3 (the device kernels' threshold) stay within the gate."""
    q, k, v = qkv(1, 256, 2048, 2, 2, seed=37, k_offset_std=0.5)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=128 ** -0.5 * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, km_bits=oracle.k_mean_bits(kb), blk=64)
    v8, vs = oracle.per_channel_fp8(vb)
    ref = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs)
    assert np.array_equal(ref, oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, lazy_tau=0.0))
    truth = oracle.attn_fp64(qb, kb, vb, 128 ** -0.5)
    for tau in (1.0, 3.0):  # 3 is the device kernels' threshold
        lazy = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, lazy_tau=tau)
        assert 0.999 < cosine(lazy, ref) < 1.0  # a different P rounding, not a different result
        assert cosine(lazy, truth) >= 0.999


def test_rounded_row_sum_mode(oracle):
    """Summing the e4m3-rounded P (as the device's MFMA row sum does) instead of the unrounded p only
    perturbs the normaliser by the fp8 rounding noise; a uniform V is then reproduced exactly up to
    the V quantization, since numerator and denominator use the same P."""
    q, k, v = qkv(1, 128, 512, 1, 1, seed=41)
    qb, kb = bf16_bits(q), bf16_bits(k)
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=128 ** -0.5 * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, blk=64)
    row = torch.linspace(-2, 2, 128).to(torch.bfloat16)
    vu = bf16_bits(row.expand(1, 512, 1, 128).contiguous())
    v8, vs = oracle.per_channel_fp8(vu)
    exact_v = oracle.e4m3_to_f32(v8[0, 0, :, 0]) * vs[0, 0]
    o = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, lsum_rounded=True)
    assert np.abs(o[0, :, 0] - exact_v[None]).max() < 1e-5
    o_ref = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs)
    assert np.abs(o_ref[0, :, 0] - exact_v[None]).max() > 1e-4  # the reference's normaliser differs


def _one_row_operands(acc, qk_mult=1.0):
    """One query row whose logits are exactly acc[j] * qk_mult (q = e0, k_j = acc[j] e0, unit scales) and
    a V that puts key j on channel j alone (e4m3 1.0), so O[j] = P_j / sum(P)."""
    n = len(acc)
    q8 = np.zeros((1, 1, 1, 128), np.int8)
    q8[0, 0, 0, 0] = 1
    k8 = np.zeros((1, n, 1, 128), np.int8)
    k8[0, :, 0, 0] = acc
    qs = np.ones((1, 1, 1), np.float32)
    ks = np.ones((1, 1, (n + 63) // 64), np.float32)
    v8 = np.zeros((1, 1, 128, 64 * ((n + 63) // 64)), np.uint8)
    for j in range(n):
        v8[0, 0, j, j] = 0x38  # e4m3 1.0
    vs = np.ones((1, 1, 128), np.float32)
    return q8, qs, k8, ks, v8, vs


def test_p_linear_known_answers(oracle):
    """p_linear: P is the e4m3 byte RNE(8 (x - 0.057539) + 56), x = s - m.  With the reference's max rule the
    top logit sits at x = 8.807: byte 126 = 448; one below, 118 = 224; 14 below, 8 * (-5.193 - 0.057539) + 56
    = 13.996 -> 14 = 2^-6 * 1.75 (the smallest normal octave); 30 below, a negative byte clamps to 0."""
    q8, qs, k8, ks, v8, vs = _one_row_operands([100, 99, 86, 70])
    o = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, lsum_rounded=True, p_linear=True)
    p = np.array([448.0, 224.0, 2.0 ** -6 * 1.75, 0.0])
    assert np.array_equal(o[0, 0, 0, :4], (p / p.sum()).astype(np.float32))
    # without p_linear the same logits give e4m3(exp2(x)): 2^8.807 = 447.9 -> 448, 2^7.807 = 223.96 -> 224,
    # 2^-5.193 = 0.02732 -> 2^-6 * 1.75 as well: the two agree on these logits
    o_ref = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, lsum_rounded=True)
    assert np.array_equal(o_ref[0, 0, 0, :4], o[0, 0, 0, :4])
    # a logit 0.5 below the top: exp2 gives 2^8.307 = 316.7 -> e4m3 320; the linear form 8 * (8.307 -
    # 0.057539) + 56 = 121.996 -> byte 122 = 2^8 * 1.25 = 320 too; 0.25 below: 2^8.557 = 376.6 -> 384,
    # linear 124 = 384
    q8, qs, k8, ks, v8, vs = _one_row_operands([100, 98, 99])
    o = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, qk_mult=0.25, lsum_rounded=True, p_linear=True)
    p = np.array([448.0, 320.0, 384.0])
    assert np.allclose(o[0, 0, 0, :3], p / p.sum(), rtol=0, atol=1e-7)


def test_p_linear_is_unbiased_and_close_to_exp2(oracle):
    """Over logits whose fractional parts cover [0, 1) evenly the linear P is exp2(x) on average within 1 %
    (the shift 0.057539 = log2(1.040685) removes the mean of (1 + f) / 2^f), its sum (weighted toward the top
    of the octave) within 2 %, and no single P leaves [-8.3 %, +8.7 %] of exp2(x) (linear interpolation error
    -4.0 / +4.4 % and the e4m3 half step of up to 6.25 %)."""
    acc = np.arange(64)  # one key tile (one running max), x spanning one octave in 1/64 steps
    q8, qs, k8, ks, v8, vs = _one_row_operands(acc)
    o, lse = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, qk_mult=1.0 / 64, lsum_rounded=True, p_linear=True,
                              want_lse=True)
    _, lse_exp = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs, qk_mult=1.0 / 64, want_lse=True)  # unrounded exp2
    assert abs(float(lse[0, 0, 0]) - float(lse_exp[0, 0, 0])) < np.log2(1.02)
    s_log = acc / 64.0
    m = s_log.max() - 8.807                      # the reference's running max
    p = o[0, 0, 0, :64].astype(np.float64) * 2.0 ** (float(lse[0, 0, 0]) - m)  # O_j * sum(P)
    rel = p / 2.0 ** (s_log - m)
    assert rel.min() > 1 - 0.083 and rel.max() < 1 + 0.087
    assert abs(rel.mean() - 1) < 0.01


# ------------------------------------------------------------------------------------------------
# per-thread quantizer (triton/quant_per_thread.py) and scale granularities of the attention oracle
# ------------------------------------------------------------------------------------------------

def test_per_thread_query_classes_closed_form(oracle):
    """Row r holds the constant r + 1: the scale of (warp block n, class c) is the largest row of the
    class, (32 n + 24 + c + 1) / 127 + 1e-7; trailing warp blocks of the 128-row padding get 1e-7."""
    L = 70
    x = np.repeat(np.arange(1, L + 1, dtype=np.float32)[:, None], 128, axis=1)
    bits = _bits(x.ravel().tolist(), (1, L, 1, 128))
    q8, qs = oracle.quant_per_thread_int8(bits)
    assert qs.shape == (1, 1, 32)
    for n in range(4):
        for c in range(8):
            rows = [32 * n + 8 * j + c for j in range(4) if 32 * n + 8 * j + c < L]
            amax = np.float32(max(rows) + 1) if rows else np.float32(0)
            want = np.float32(np.float32(amax / np.float32(127.0)) + np.float32(1e-7))
            assert qs[0, 0, n * 8 + c] == want, (n, c)
    # the largest row of every class quantizes to 127 (x / scale just below 127, rounds half away)
    for c in range(8):
        top = max(r for r in range(L) if r % 8 == c)  # the largest row of its class and warp block
        assert q8[0, top, 0, 0] == 127


def test_per_thread_key_classes_closed_form(oracle):
    """Key class c of a 64-row block holds rows 8j + 2c and 8j + 2c + 1 (mma lane pairs)."""
    L = 64
    x = np.repeat(np.arange(1, L + 1, dtype=np.float32)[:, None], 128, axis=1)
    k8, ks = oracle.quant_per_thread_int8(_bits(x.ravel().tolist(), (1, L, 1, 128)), is_key=True)
    assert ks.shape == (1, 1, 4)
    for c in range(4):
        want = np.float32(np.float32(np.float32(56 + 2 * c + 2) / np.float32(127.0)) + np.float32(1e-7))
        assert ks[0, 0, c] == want
    assert (k8[0, 56 + 2 * np.arange(4) + 1, 0, :] == 127).all()


def test_per_thread_zero_rows_and_half_away(oracle):
    x = np.zeros((1, 32, 1, 128), np.float32)
    x[0, 1, 0, :3] = [2.0, -2.0, 1.0]  # class 1: amax 2 -> scale 2/127 + 1e-7
    q8, qs = oracle.quant_per_thread_int8(bf16_bits(torch.from_numpy(x)))
    assert qs[0, 0, 0] == np.float32(1e-7) and (q8[0, 0] == 0).all()
    sc = np.float32(np.float32(2.0 / np.float32(127.0)) + np.float32(1e-7))
    t = np.float32(1.0) / sc  # 63.4999968...: half-away keeps 63
    assert q8[0, 1, 0, 0] == 127 and q8[0, 1, 0, 1] == -127 and q8[0, 1, 0, 2] == int(np.trunc(t + 0.5))


@pytest.mark.parametrize("L,is_key,sm90", [(300, False, False), (300, True, False), (1000, True, False),
                                           (129, False, False), (300, False, True), (300, True, True),
                                           (1000, True, True), (129, False, True), (40, False, True)])
def test_per_thread_random_matches_numpy_restatement(oracle, L, is_key, sm90):
    """Vectorised float32 numpy version with the class mapping built by reshapes (not index formulas).
    sm90: 16-row query warp blocks in 64-row CTA blocks, 128-row key blocks (sageattn2.py:1614-1624)."""
    g = torch.Generator().manual_seed(L)
    x = (torch.randn((2, L, 3, 128), generator=g) * 2).to(torch.bfloat16)
    km = (torch.randn((2, 1, 3, 128), generator=g)).to(torch.bfloat16) if is_key else None
    xd = (x - km) if is_key else x  # torch bf16 op, as the reference wrapper does
    q8, sc = oracle.quant_per_thread_int8(bf16_bits(x), None if km is None else bf16_bits(km[:, 0]), is_key=is_key,
                                          sm90=sm90)
    xf = xd.float().numpy()
    if sm90:
        blk = 128 if is_key else 16
        nb = -(-L // 128) if is_key else -(-L // 64) * 4
    else:
        blk = 64 if is_key else 32
        nb = -(-L // 64) if is_key else -(-L // 128) * 4
    pad = np.zeros((2, nb * blk, 3, 128), np.float32)
    pad[:, :L] = xf
    if is_key:  # [b, n, j(blk/8), cls(4), pair(2), h, d]
        v = pad.reshape(2, nb, blk // 8, 4, 2, 3, 128)
        amax = np.abs(v).max(axis=(2, 4, 6))                 # [b, n, cls, h]
    else:       # [b, n, j(blk/8), cls(8), h, d]
        v = pad.reshape(2, nb, blk // 8, 8, 3, 128)
        amax = np.abs(v).max(axis=(2, 5))
    scale = (amax / np.float32(127.0) + np.float32(1e-7)).astype(np.float32)
    want_sc = scale.transpose(0, 3, 1, 2).reshape(2, 3, -1)
    assert np.array_equal(sc, want_sc)
    if is_key:
        sfull = np.broadcast_to(scale[:, :, None, :, None, :, None], v.shape).reshape(2, nb * blk, 3, 128)
    else:
        sfull = np.broadcast_to(scale[:, :, None, :, :, None], v.shape).reshape(2, nb * blk, 3, 128)
    t = (pad / sfull).astype(np.float32)
    want = np.trunc(t + np.where(t >= 0, 0.5, -0.5).astype(np.float32)).astype(np.int8)[:, :L]
    assert np.array_equal(q8, want)


def test_attention_oracle_granularity_indexing(oracle):
    """Per-warp / per-thread scales fed as expanded per-block-equivalent data give the same O: a tensor
    whose scales are constant inside every 128-query / 64-key block must not depend on the granularity."""
    q, k, v = qkv(1, 200, 300, 2, 1, seed=11)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=128 ** -0.5 * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, blk=64)
    v8, vs = oracle.per_channel_fp8(vb)
    base = oracle.qattn_fwd(q8, qs, k8, ks, v8, vs)
    qs_w = np.repeat(qs, 4, axis=-1)           # 4 warps per 128-row block
    qs_t = np.repeat(qs_w, 8, axis=-1)         # 8 lane classes per warp
    ks_t = np.repeat(ks, 4, axis=-1)           # 4 lane-pair classes per key block
    for qg, qsg in ((2, qs_w), (3, qs_t)):
        for kg, ksg in ((1, ks), (3, ks_t)):
            o = oracle.qattn_fwd(q8, qsg, k8, ksg, v8, vs, q_gran=qg, k_gran=kg)
            assert np.array_equal(o, base), (qg, kg)
    # and a scale change in one class touches exactly the rows / keys of that class
    qs_t2 = qs_t.copy()
    qs_t2[0, 0, 3] *= 2.0  # warp block 0, class 3: rows 3, 11, 19, 27 of head 0
    o2 = oracle.qattn_fwd(q8, qs_t2, k8, ks, v8, vs, q_gran=3, k_gran=1)
    changed = np.nonzero(np.abs(o2 - base).max(axis=-1) > 0)
    assert sorted(set(zip(changed[1].tolist(), changed[2].tolist()))) == [(3, 0), (11, 0), (19, 0), (27, 0)]
    ks_t2 = ks_t.copy()
    ks_t2[0, 0, 4 + 2] *= 0.25  # key block 1, class 2: keys 64 + 8j + 4, 64 + 8j + 5 only
    o3 = oracle.qattn_fwd(q8, qs, k8, ks_t2, v8, vs, q_gran=1, k_gran=3)
    sel = [64 + 8 * j + 4 + e for j in range(8) for e in range(2)]
    # against a direct float64 softmax over the dequantized logits with that class rescaled
    qf = q8[0, :, 0].astype(np.float64) * np.repeat(qs[0, 0], 128)[:200, None]
    kscale = np.repeat(ks[0, 0], 64)[:300].astype(np.float64)
    kscale[sel] *= 0.25
    kf = k8[0, :, 0].astype(np.float64) * kscale[:, None]
    s = qf @ kf.T
    p = np.exp2(s - s.max(axis=1, keepdims=True))
    vf = oracle.e4m3_to_f32(v8[0, 0, :, :300]).T.astype(np.float64) * vs[0, 0][None, :]
    ref = (p @ vf) / p.sum(axis=1, keepdims=True)
    assert cosine(o3[0, :, 0], ref) > 0.9995


def test_sm90_per_thread_tables_refine_sm89(oracle):
    """The sm89 and sm90 per-thread tables partition the same rows into nested cells: an sm89 query cell
    (32-row warp, class c) is the union of the sm90 cells (two 16-row warps, class c), and an sm90 key
    cell (128-row block, class c) the union of two sm89 ones (64-row blocks).  scale = amax / 127 + 1e-7
    is monotone in amax, so the coarser cell's scale is the maximum of its parts' scales exactly."""
    g = torch.Generator().manual_seed(5)
    L = 333
    x = (torch.randn((1, L, 2, 128), generator=g) * torch.linspace(0.2, 3.0, L)[None, :, None, None])
    xb = bf16_bits(x.to(torch.bfloat16))
    _, q89 = oracle.quant_per_thread_int8(xb)
    _, q90 = oracle.quant_per_thread_int8(xb, sm90=True)
    _, k89 = oracle.quant_per_thread_int8(xb, is_key=True)
    _, k90 = oracle.quant_per_thread_int8(xb, is_key=True, sm90=True)
    assert q89.shape == (1, 2, 3 * 32) and q90.shape == (1, 2, 6 * 32)
    assert k89.shape == (1, 2, 6 * 4) and k90.shape == (1, 2, 3 * 4)
    q90w = q90.reshape(1, 2, -1, 2, 8)                     # [b, h, 32-row warp, half, class]
    assert np.array_equal(q89.reshape(1, 2, -1, 8), q90w.max(axis=3))
    k89b = k89.reshape(1, 2, -1, 2, 4)                     # [b, h, 128-row block, half, class]
    assert np.array_equal(k90.reshape(1, 2, -1, 4), k89b.max(axis=3))


def test_attention_oracle_sm90_indexing(oracle):
    """q_gran / k_gran 4, 5 (the sm90 tables): scale tables that give every row the same scale as an sm89
    table give the same O, and a change in one sm90 cell touches exactly the rows / keys of that cell."""
    q, k, v = qkv(1, 200, 300, 2, 1, seed=12)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    q8, _ = oracle.quant_per_thread_int8(qb)
    k8, _ = oracle.quant_per_thread_int8(kb, is_key=True)
    v8, vs = oracle.per_channel_fp8(vb)
    rng = np.random.default_rng(3)
    # per-row scale functions: query f(row // 32, row % 8), key g(key // 128, (key % 8) // 2)
    fq = rng.uniform(0.01, 0.03, size=(2, 7, 8)).astype(np.float32)   # [head, row // 32, row % 8]
    fk = rng.uniform(0.01, 0.03, size=(1, 3, 4)).astype(np.float32)   # [kv head, key // 128, class]
    qs89 = np.zeros((1, 2, 2 * 32), np.float32)                        # ceil(200/128) = 2 blocks x 32
    qs90 = np.zeros((1, 2, 4 * 32), np.float32)                        # ceil(200/64) = 4 blocks x 32
    for w in range(8):                     # 32-row warps of the sm89 table
        qs89[0, :, w * 8:(w + 1) * 8] = fq[:, min(w, 6)]
    for w in range(16):                    # 16-row warps of the sm90 table
        qs90[0, :, w * 8:(w + 1) * 8] = fq[:, min(w // 2, 6)]
    ks89 = np.zeros((1, 1, 5 * 4), np.float32)                         # ceil(300/64) = 5 blocks x 4
    ks90 = np.zeros((1, 1, 3 * 4), np.float32)                         # ceil(300/128) = 3 blocks x 4
    for t in range(5):
        ks89[0, :, t * 4:(t + 1) * 4] = fk[:, t // 2]
    for t in range(3):
        ks90[0, :, t * 4:(t + 1) * 4] = fk[:, t]
    qk = 128 ** -0.5 * LOG2E
    base = oracle.qattn_fwd(q8, qs89, k8, ks89, v8, vs, qk_mult=qk, q_gran=3, k_gran=3)
    o = oracle.qattn_fwd(q8, qs90, k8, ks90, v8, vs, qk_mult=qk, q_gran=5, k_gran=5)
    assert np.array_equal(o, base)
    # per-warp: one scale per 16-row warp / 128-key block
    qw89 = fq[None, :, [min(w, 6) for w in range(8)], 0]
    qw90 = fq[None, :, [min(w // 2, 6) for w in range(16)], 0]
    kw89 = fk[None, :, [t // 2 for t in range(5)], 0]
    kw90 = fk[None, :, :, 0]
    base_w = oracle.qattn_fwd(q8, np.ascontiguousarray(qw89), k8, np.ascontiguousarray(kw89), v8, vs, qk_mult=qk,
                              q_gran=2, k_gran=2)
    o_w = oracle.qattn_fwd(q8, np.ascontiguousarray(qw90), k8, np.ascontiguousarray(kw90), v8, vs, qk_mult=qk,
                           q_gran=4, k_gran=4)
    assert np.array_equal(o_w, base_w)
    # one sm90 query cell: 16-row warp 3, class 5 = rows 53, 61 of head 1
    qs2 = qs90.copy()
    qs2[0, 1, 3 * 8 + 5] *= 2.0
    o2 = oracle.qattn_fwd(q8, qs2, k8, ks90, v8, vs, qk_mult=qk, q_gran=5, k_gran=5)
    changed = np.nonzero(np.abs(o2 - o).max(axis=-1) > 0)
    assert sorted(set(zip(changed[1].tolist(), changed[2].tolist()))) == [(53, 1), (61, 1)]
    # one sm90 key cell: 128-key block 1, class 3 = keys 128 + 8j + 6, 128 + 8j + 7: the logits of
    # exactly those keys scale (against a float64 softmax over the dequantized logits)
    ks2 = ks90.copy()
    ks2[0, 0, 4 + 3] *= 0.25
    o3 = oracle.qattn_fwd(q8, qs90, k8, ks2, v8, vs, qk_mult=qk, q_gran=5, k_gran=5)
    rows = np.arange(200)
    qrow_scale = qs90[0, 0][(rows // 16) * 8 + rows % 8].astype(np.float64)
    keys = np.arange(300)
    kscale = fk[0][keys // 128, (keys % 8) // 2].astype(np.float64)
    kscale[[128 + 8 * j + 6 + e for j in range(16) for e in range(2)]] *= 0.25
    s = (q8[0, :, 0].astype(np.float64) * qrow_scale[:, None]) @ (k8[0, :, 0].astype(np.float64)
                                                                * kscale[:, None]).T * qk
    p = np.exp2(s - s.max(axis=1, keepdims=True))
    vf = oracle.e4m3_to_f32(v8[0, 0, :, :300]).T.astype(np.float64) * vs[0, 0][None, :]
    ref = (p @ vf) / p.sum(axis=1, keepdims=True)
    assert cosine(o3[0, :, 0], ref) > 0.9995


def test_block_sparse_tile_mask(oracle):
    """A skipped key tile is exactly a tile removed from K, V and the key scales
    (sparse_int8_attn.py:57-58); an all-ones mask is the dense computation; a fully masked query block
    gives zeros."""
    q, k, v = qkv(1, 256, 384, 2, 2, seed=12, k_offset_std=0.5)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    q8, qs = oracle.quant_per_block_int8(qb, sm_scale=128 ** -0.5 * LOG2E, blk=128)
    k8, ks = oracle.quant_per_block_int8(kb, blk=64)
    vh = vb  # bf16 V, half P.V (the sparse kernel's mode)
    dense = oracle.qattn_fwd(q8, qs, k8, ks, vh_bits=vh, pv_mode=1)
    ones = np.ones((1, 2, 2, 6), np.int8)
    assert np.array_equal(oracle.qattn_fwd(q8, qs, k8, ks, vh_bits=vh, pv_mode=1, tile_mask=ones), dense)
    mask = ones.copy()
    mask[0, :, 0, 2] = 0  # query block 0 skips keys 128..191 in both heads
    mask[0, 1, 1, :] = 0  # head 1, query block 1: nothing
    got = oracle.qattn_fwd(q8, qs, k8, ks, vh_bits=vh, pv_mode=1, tile_mask=mask)
    keep = np.r_[0:128, 192:384]
    ref = oracle.qattn_fwd(q8[:, :128], qs[:, :, :1], np.ascontiguousarray(k8[:, keep]),
                           np.ascontiguousarray(ks[:, :, [0, 1, 3, 4, 5]]), vh_bits=np.ascontiguousarray(vh[:, keep]),
                           pv_mode=1)
    assert np.array_equal(got[:, :128], ref)
    assert np.array_equal(got[:, 128:, 0], dense[:, 128:, 0])
    assert not got[:, 128:, 1].any()


# ------------------------------------------------------------------------------------------------
# RMSNorm + RoPE prologue (norm.py:469-507, rotary.py:21-88)
# ------------------------------------------------------------------------------------------------

def _norm_rope_inputs(L=40, H=2, D=128, seed=3):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((1, L, H * D), generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn((H * D,), generator=g)).to(torch.bfloat16)
    ang = torch.rand((L, D // 2), generator=g, dtype=torch.float64) * 6.3
    return x, w, ang.cos().float().numpy(), ang.sin().float().numpy()


def test_norm_rope_known_answers(oracle):
    D = 128
    # constant row 2.0, unit weight, no rotation: var = 4, y = bf16(2 / sqrt(4 + 1e-6)) = 1.0
    x = np.full((1, 1, 2 * D), 0x4000, np.uint16)  # bf16 2.0
    w = np.full((2 * D,), 0x3F80, np.uint16)       # bf16 1.0
    one, zero = np.ones((1, D // 2), np.float32), np.zeros((1, D // 2), np.float32)
    out = oracle.norm_rope(x, w, one, zero, D)
    assert (out == 0x3F80).all()
    # a quarter turn maps each pair (y1, y2) to (-y2, y1) exactly
    xb, wb, _, _ = _norm_rope_inputs(L=3)
    c0, s1 = np.zeros((3, D // 2), np.float32), np.ones((3, D // 2), np.float32)
    plain = oracle.norm_rope(bf16_bits(xb), bf16_bits(wb), np.ones_like(c0), c0, D)
    turned = oracle.norm_rope(bf16_bits(xb), bf16_bits(wb), c0, s1, D)
    pf, tf = oracle.bf16_bits_to_f32(plain), oracle.bf16_bits_to_f32(turned)
    assert np.array_equal(tf[..., 0::2], -pf[..., 1::2]) and np.array_equal(tf[..., 1::2], pf[..., 0::2])


def test_norm_rope_scale_invariance_and_torch(oracle):
    """RMSNorm is invariant to scaling the row by a power of two (exactly, in floating point); the output
    agrees with a float32 torch restatement of the two Triton kernels (whose only difference is the
    reduction order of the mean of squares) on all but a handful of bf16 values, by at most one ulp."""
    D = 128
    x, w, cs, sn = _norm_rope_inputs()
    a = oracle.norm_rope(bf16_bits(x), bf16_bits(w), cs, sn, D)
    b = oracle.norm_rope(bf16_bits(x * 8), bf16_bits(w), cs, sn, D)
    assert np.array_equal(a, b)
    xf = x.float()
    rstd = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    y = ((xf * rstd) * w.float()).to(torch.bfloat16).float().reshape(1, 40, 2, D // 2, 2)
    c, s = torch.from_numpy(cs)[None, :, None, :], torch.from_numpy(sn)[None, :, None, :]
    o1 = torch.addcmul(y[..., 0] * c, -y[..., 1], s)
    o2 = torch.addcmul(y[..., 1] * c, y[..., 0], s)
    ref = bf16_bits(torch.stack([o1, o2], -1).reshape(1, 40, 2 * D))
    diff = np.abs(oracle.bf16_bits_to_f32(a) - oracle.bf16_bits_to_f32(ref))
    rel = diff / np.maximum(np.abs(oracle.bf16_bits_to_f32(ref)), 1e-30)
    assert (a != ref).mean() < 0.01
    assert rel.max() <= 2 ** -7
