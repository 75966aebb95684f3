"""QuantizedKVCache on the GPU: the cache state after every streaming step is the oracle's quantization of
its bf16 slots (bit-exact), and each step's output matches attention over the reference's window
(telefuser/models/lingbot_world_fast_dit.py:147-187: roll, append, non-causal attention())."""

import numpy as np
import pytest
import torch

from tests.gpu_util import log, require_gpu, untile_v
from tests.inputs import bf16_bits, cosine

pytestmark = pytest.mark.gpu

COS_KERNEL = 0.99995
COS_E2E = 0.999


def _check_state(oracle, cache, v_seen_amax):
    """k8 / k_scale / v8 / v_scale over slots [0, high_water) against the oracle, bit for bit."""
    hw = cache.high_water
    k16 = bf16_bits(cache.k16[:, :hw].cpu())
    km = bf16_bits(cache.k_mean.cpu())
    k8_ref, ks_ref = oracle.quant_per_block_int8(k16, km, None, blk=64)
    assert np.array_equal(cache.k8[:, :hw].cpu().numpy(), k8_ref)
    nblk = ks_ref.shape[-1]
    assert np.array_equal(cache.k_scale[:, :, :nblk].cpu().numpy(), ks_ref)
    amax = cache.v_amax.cpu().numpy()
    assert np.array_equal(amax, v_seen_amax)
    assert np.array_equal(cache.v_scale.cpu().numpy(), amax / np.float32(448.0))
    v = oracle.bf16_bits_to_f32(bf16_bits(cache.v16[:, :hw].cpu()))  # [B, hw, H, D]
    recp = (np.float32(448.0) / amax)[:, None]                       # [B, 1, H, D]
    want = oracle.cvt_array((v * recp).astype(np.float32), "e4m3").transpose(0, 2, 3, 1)
    got = untile_v(cache.v8)[..., :hw]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("size,sink,n,local_attn,repeats", [
    (1000, 200, 200, 5, 2),   # rolls with sink tokens, chunks not block aligned, each chunk run twice
    (768, 0, 256, 3, 1),      # block-aligned ring
])
def test_cache_state_and_output(oracle, size, sink, n, local_attn, repeats):
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa
    from telefuser_amd.kv_cache import QuantizedKVCache

    B, H, D = 1, 2, 128
    g = torch.Generator().manual_seed(size + n)
    cache = QuantizedKVCache(B, size, H, D, sink_tokens=sink, device=dev)
    ref_k = torch.zeros(B, size, H, D, dtype=torch.bfloat16)
    ref_v = torch.zeros_like(ref_k)
    seen = np.zeros((B, H, D), np.float32)
    step = 0
    for c in range(8):
        for r in range(repeats):
            start = c * n
            q, k, v = (torch.randn((B, n, H, D), generator=g).to(torch.bfloat16) for _ in range(3))
            k = k + 0.7  # a channel bias for the smoothing to remove
            if c == 5 and r == 0:
                v = v * 3.0  # forces a per-channel amax growth: full V re-encode
            log(f"kv-cache size={size} sink={sink} n={n} step={step} start={start}")
            seen = np.maximum(seen, np.abs(v.float().numpy()).max(axis=1))
            o = cache.step(q.to(dev), k.to(dev), v.to(dev), start, sink_tokens=sink, local_attn_size=local_attn)
            torch.cuda.synchronize()
            _check_state(oracle, cache, seen)
            # the reference cache window, maintained on the CPU exactly as the reference does
            le = cache.local_end
            idx = cache.window_slots(0, le)
            wk, wv = cache.k16[:, idx.to(dev)].cpu(), cache.v16[:, idx.to(dev)].cpu()
            truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(wk), bf16_bits(wv), D ** -0.5)
            og = o.float().cpu().numpy()
            ct = cosine(og, truth)
            # same quantized operands through the oracle's attention (kernel schedule)
            q8, qs = sa.quant_per_block_int8(q.to(dev), 128, sm_scale=D ** -0.5 * sa.LOG2E, tensor_layout="NHD")
            kv_valid = [le] if le < size else None
            L = __import__("telefuser_amd._lib", fromlist=["load"]).load()
            ns = min(L.qattn_fwd_num_splits(B, n, size, H), (size + 63) // 64)
            tps = ((size + 63) // 64 + ns - 1) // ns if ns > 1 else 0
            ref = oracle.qattn_fwd(q8.cpu().numpy(), qs.cpu().numpy(), cache.k8.cpu().numpy(),
                                   cache.k_scale.cpu().numpy(), v8=untile_v(cache.v8), v_scale=cache.v_scale.cpu().numpy(),
                                   kv_valid=kv_valid, tiles_per_split=tps, lazy_tau=3.0, lsum_rounded=True,
                                   p_linear=True)
            ck = cosine(og, ref)
            log(f"  local_end={le} head={cache.head} cos_truth={ct:.6f} cos_oracle={ck:.6f}")
            assert ct >= COS_E2E
            assert ck >= COS_KERNEL
            step += 1


def test_cache_lse_and_fallback_window(oracle):
    """return_lse adds back the frozen-mean correction; a window shorter than the cache takes the gathered path."""
    dev = require_gpu()
    from telefuser_amd.kv_cache import QuantizedKVCache

    B, H, D, n = 1, 2, 128, 192
    g = torch.Generator().manual_seed(7)
    cache = QuantizedKVCache(B, 4 * n, H, D, device=dev)
    for c in range(3):
        q, k, v = (torch.randn((B, n, H, D), generator=g).to(torch.bfloat16) for _ in range(3))
        o, lse = cache.step(q.to(dev), (k + 0.5).to(dev), v.to(dev), c * n, return_lse=True)
    le = cache.local_end
    wk, wv = cache.k16[:, :le].cpu(), cache.v16[:, :le].cpu()
    s = torch.einsum("bqhd,bkhd->bhqk", q.double(), wk.double()) * D ** -0.5
    lse_true = torch.logsumexp(s, dim=-1).numpy()
    assert float(np.abs(lse.cpu().numpy() - lse_true).max()) < 0.05
    # window of the last 2n positions only: reference-ordered gather + attention()
    q, k, v = (torch.randn((B, n, H, D), generator=g).to(torch.bfloat16) for _ in range(3))
    o = cache.step(q.to(dev), k.to(dev), v.to(dev), 3 * n, max_attention_size=2 * n)
    wk, wv = cache.k16[:, 2 * n:4 * n].cpu(), cache.v16[:, 2 * n:4 * n].cpu()
    truth = oracle.attn_fp64(bf16_bits(q), bf16_bits(wk), bf16_bits(wv), D ** -0.5)
    assert cosine(o.float().cpu().numpy(), truth) >= COS_E2E
