"""HIP graph capture of the drop-in calls: the path allocates nothing outside torch's graph pool, reads
no device value on the host and uses no memset, so a captured call replays correctly.  Each replay runs
on fresh inputs copied into the captured tensors, with eager calls of the same op in between, and must
equal the eager result bit for bit."""

import pytest
import torch

from tests.gpu_util import log, require_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kw", [
    dict(qk_quant_gran="per_thread", pv_accum_dtype="fp32+fp32"),   # TeleFuser's call
    dict(qk_quant_gran="per_warp", pv_accum_dtype="fp32", smooth_v=True),
    dict(qk_quant_gran="per_thread", pv_accum_dtype="fp32+fp16"),
])
def test_sageattn_graph_replay_matches_eager(kw):
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    B, L, H, D = 1, 1500, 4, 128
    g = torch.Generator(device=dev).manual_seed(5)
    mk = lambda: torch.randn((B, L, H, D), generator=g, device=dev).to(torch.bfloat16)
    q, k, v = mk(), mk(), mk()
    call = lambda: sa.sageattn_qk_int8_pv_fp8_cuda(q, k, v, tensor_layout="NHD", **kw)
    log(f"graph capture {kw}")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            call()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for rep in range(3):
        for t in (q, k, v):
            t.copy_(mk())
        graph.replay()
        ref = call()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from the eager call"


def test_varlen_graph_replay_matches_eager():
    dev = require_gpu()
    from telefuser_amd import sageattn2 as sa

    H, D = 2, 128
    lq, lk = [300, 0, 257], [130, 64, 600]
    cq = torch.tensor([0, 300, 300, 557], dtype=torch.int32, device=dev)
    ck = torch.tensor([0, 130, 194, 794], dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(6)
    q = torch.randn((557, H, D), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((794, H, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((794, H, D), generator=g, device=dev).to(torch.bfloat16)
    call = lambda: sa.sageattn_varlen(q, k, v, cq, ck, max(lq), max(lk))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            call()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for rep in range(3):
        q.copy_(torch.randn(q.shape, generator=g, device=dev).to(torch.bfloat16))
        k.copy_(torch.randn(k.shape, generator=g, device=dev).to(torch.bfloat16))
        graph.replay()
        ref = call()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from the eager call"
