"""qattn_fwd_ex_noalloc (KV-split partials in the library's own device array, no allocation) against
qattn_fwd_ex with a caller workspace, through the C ABI: identical output and LSE bits on two calls in a
row (the second smaller, so stale scratch contents from the first would show), and the size limit."""

import pytest
import torch

from tests.gpu_util import log, require_gpu
from tests.inputs import qkv

pytestmark = pytest.mark.gpu


def _quantized(dev, B, Lq, Lk, H, seed, D=128):
    from telefuser_amd import sageattn2 as sa

    q, k, v = qkv(B, Lq, Lk, H, H, D=D, seed=seed, k_offset_std=0.5)
    q, k, v = (t.to(dev) for t in (q, k, v))
    km = sa.k_mean(k, "NHD")
    q8, qs, k8, ks = sa.per_block_int8(q, k, km, sm_scale=D ** -0.5, tensor_layout="NHD")
    v8, vs, _ = sa.per_channel_fp8(v, tensor_layout="NHD", smooth_v=False)
    return q8, qs, k8, ks, v8, vs


def _call(noalloc, t, B, Lq, Lk, H, splits, kv_valid, stream=None):
    from telefuser_amd import _lib

    L = _lib.load()
    q8, qs, k8, ks, v8, vs = t
    dev = q8.device
    D = q8.shape[-1]
    o = torch.empty(q8.shape, dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, H, Lq), dtype=torch.float32, device=dev)
    kvv = None if kv_valid is None else torch.tensor(kv_valid, dtype=torch.int32, device=dev)
    args = (_lib.seq(q8, "NHD"), _lib.ptr(qs), _lib.seq(k8, "NHD"), _lib.ptr(ks), _lib.ptr(v8), _lib.QATTN_V_FP8,
            v8.shape[-1], _lib.ptr(vs), _lib.seq(o, "NHD"), _lib.QATTN_BF16, B, Lq, Lk, H, H, D, 1.0,
            _lib.QATTN_GRAN_BLOCK, 0, 0, _lib.ptr(kvv), _lib.ptr(lse), splits)
    if noalloc:
        st = _lib.stream_of(q8) if stream is None else stream.cuda_stream
        _lib.check(L.qattn_fwd_ex_noalloc(*args, st))
    else:
        ns = splits if splits > 0 else L.qattn_fwd_ex_num_splits(B, Lq, Lk, H, 0, 1)
        wsb = L.qattn_fwd_workspace_size(B, Lq, H, D, ns)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
        _lib.check(L.qattn_fwd_ex(*args[:-1], ns, _lib.ptr(ws), wsb, _lib.stream_of(q8)))
    return o, lse


def test_noalloc_matches_workspace_entry_twice():
    dev = require_gpu()
    from telefuser_amd import _lib

    L = _lib.load()
    cases = [  # (B, Lq, Lk, H, splits, kv_valid): a C5-length chunk on 2 heads with its automatic split
        (1, 4680, 32760, 2, 0, None),  # (38 pairs: 6 splits, ping-pong), then a smaller launch
        (2, 700, 9000, 3, 5, [9000, 4100]),
    ]
    for i, (B, Lq, Lk, H, splits, kvv) in enumerate(cases):
        ns = splits if splits > 0 else L.qattn_fwd_ex_num_splits(B, Lq, Lk, H, 0, 1)
        log(f"noalloc call {i}: B={B} Lq={Lq} Lk={Lk} H={H} splits={ns} kv_valid={kvv}")
        assert ns > 1
        assert L.qattn_fwd_workspace_size(B, Lq, H, 128, ns) <= L.qattn_fwd_noalloc_max_scratch()
        t = _quantized(dev, B, Lq, Lk, H, seed=300 + i)
        o0, l0 = _call(False, t, B, Lq, Lk, H, splits, kvv)
        o1, l1 = _call(True, t, B, Lq, Lk, H, splits, kvv)
        torch.cuda.synchronize()
        assert torch.equal(o0, o1), f"call {i}: max diff {float((o0.float() - o1.float()).abs().max())}"
        assert torch.equal(l0, l1)
        assert bool(torch.isfinite(o1.float()).all())


def test_noalloc_rejects_launch_beyond_scratch():
    dev = require_gpu()
    from telefuser_amd import _lib

    L = _lib.load()
    B, Lq, Lk, H, splits = 1, 32760, 32760, 12, 32  # 32 splits x 12 x 32760 x 130 x 4 B = 6.5 GB of partials
    assert L.qattn_fwd_workspace_size(B, Lq, H, 128, splits) > L.qattn_fwd_noalloc_max_scratch()
    q8 = torch.zeros((B, Lq, H, 128), dtype=torch.int8, device=dev)
    k8 = torch.zeros((B, Lk, H, 128), dtype=torch.int8, device=dev)
    v8 = torch.zeros((B, H, 128, Lk // 64 * 64 + 64), dtype=torch.uint8, device=dev)
    sc = torch.ones((B, H, 512), dtype=torch.float32, device=dev)
    o = torch.empty((B, Lq, H, 128), dtype=torch.bfloat16, device=dev)
    rc = L.qattn_fwd_ex_noalloc(_lib.seq(q8, "NHD"), _lib.ptr(sc), _lib.seq(k8, "NHD"), _lib.ptr(sc), _lib.ptr(v8),
                                0, v8.shape[-1], _lib.ptr(sc), _lib.seq(o, "NHD"), 0, B, Lq, Lk, H, H, 128, 1.0, 1, 0,
                                0, None, None, splits, _lib.stream_of(q8))
    assert rc == 7, rc  # QATTN_ERR_WORKSPACE, before any launch
    assert "scratch" in L.qattn_last_error().decode()


def test_noalloc_calls_on_two_streams_are_ordered():
    """Two KV-split launches issued back to back on two streams, with no host synchronisation between them:
    the second waits on the GPU for the first one's use of the shared scratch, so both outputs equal the
    workspace entry's bit for bit."""
    dev = require_gpu()
    from telefuser_amd import _lib

    L = _lib.load()
    cases = [(1, 4680, 32760, 2, 0, None), (1, 2000, 20000, 2, 6, None)]
    data = []
    for i, (B, Lq, Lk, H, splits, kvv) in enumerate(cases):
        ns = splits if splits > 0 else L.qattn_fwd_ex_num_splits(B, Lq, Lk, H, 0, 1)
        log(f"two-stream noalloc call {i}: B={B} Lq={Lq} Lk={Lk} H={H} splits={ns}")
        assert ns > 1
        t = _quantized(dev, B, Lq, Lk, H, seed=400 + i)
        data.append((t, _call(False, t, B, Lq, Lk, H, splits, kvv)))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for (t, _), (B, Lq, Lk, H, splits, kvv), st in zip(data, cases, streams):
        outs.append(_call(True, t, B, Lq, Lk, H, splits, kvv, stream=st))
    torch.cuda.synchronize()
    for i, ((_, (o0, l0)), (o1, l1)) in enumerate(zip(data, outs)):
        assert torch.equal(o0, o1), f"stream {i}: max diff {float((o0.float() - o1.float()).abs().max())}"
        assert torch.equal(l0, l1)


def test_noalloc_head_dim_64():
    """The allocation-free entry on the head-dim-64 form (KV split through the in-library scratch), twice,
    bit-identical to the workspace entry."""
    dev = require_gpu()
    from telefuser_amd import _lib

    L = _lib.load()
    for i, (B, Lq, Lk, H, splits) in enumerate([(1, 2000, 16000, 4, 0), (1, 600, 5000, 2, 3)]):
        ns = splits if splits > 0 else L.qattn_fwd_ex_num_splits(B, Lq, Lk, H, 0, 1)
        log(f"noalloc head_dim 64 call {i}: B={B} Lq={Lq} Lk={Lk} H={H} splits={ns}")
        assert ns > 1
        t = _quantized(dev, B, Lq, Lk, H, seed=500 + i, D=64)
        o0, l0 = _call(False, t, B, Lq, Lk, H, splits, None)
        o1, l1 = _call(True, t, B, Lq, Lk, H, splits, None)
        torch.cuda.synchronize()
        assert torch.equal(o0, o1) and torch.equal(l0, l1)
        assert bool(torch.isfinite(o1.float()).all())
