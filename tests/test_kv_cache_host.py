"""Host bookkeeping of the streaming KV cache (CPU): the ring-ordered QuantizedKVCache must hold, for every
step, exactly the keys/values of the reference's rolling bf16 cache window
(telefuser/models/lingbot_world_fast_dit.py:147-187), which streaming_self_attention reproduces on a dict."""

import pytest
import torch

from telefuser_amd.attention import AttentionConfig, AttnImplType
from telefuser_amd.kv_cache import QuantizedKVCache, streaming_self_attention

SDPA = AttentionConfig(attn_impl=AttnImplType.TORCH_SDPA)


def _schedule(n_chunks, n, repeats):
    for c in range(n_chunks):
        for _ in range(repeats):
            yield c * n


@pytest.mark.parametrize("size,sink,n,local_attn,repeats", [
    (300, 70, 50, 6, 2),     # rolling with sink tokens, each chunk denoised twice
    (320, 0, 64, 5, 1),      # block-aligned, no sink
    (400, 0, 37, -1, 3),     # no rolling (local_attn_size = -1), cache never full
    (257, 100, 40, 3, 2),    # odd sizes, sink larger than a chunk
])
def test_ring_cache_matches_reference_window(size, sink, n, local_attn, repeats):
    torch.manual_seed(size)
    B, H, D = 1, 2, 128
    ref = {"k": torch.zeros(B, size, H, D), "v": torch.zeros(B, size, H, D),
           "global_end_index": torch.tensor(0), "local_end_index": torch.tensor(0)}
    cache = QuantizedKVCache(B, size, H, D, sink_tokens=sink, dtype=torch.float32, device="cpu")
    n_chunks = 12 if local_attn != -1 else size // n
    for start in _schedule(n_chunks, n, repeats):
        q, k, v = (torch.randn(B, n, H, D) for _ in range(3))
        out = streaming_self_attention(q, k, v, ref, start, sink_tokens=sink, local_attn_size=local_attn,
                                       attention_config=SDPA)
        ranges, local_end = cache.advance(k, v, start, local_attn)
        assert local_end == int(ref["local_end_index"])
        assert sum(e - a for a, e in ranges) == n
        idx = cache.window_slots(0, local_end)
        assert torch.equal(cache.k16[:, idx], ref["k"][:, :local_end])
        assert torch.equal(cache.v16[:, idx], ref["v"][:, :local_end])
        # the window is a prefix of slots whenever the step would take the fast path
        if cache.head == 0 or local_end == size:
            assert sorted(idx.tolist()) == list(range(local_end))
        assert cache.high_water >= local_end
        assert out.shape == q.shape


def test_ring_rejects_gaps():
    cache = QuantizedKVCache(1, 256, 1, 128, dtype=torch.float32, device="cpu")
    x = torch.zeros(1, 64, 1, 128)
    cache.advance(x, x, 0)
    with pytest.raises(ValueError, match="gap"):
        cache.advance(x, x, 200)  # the reference would attend to never-written zeros


def test_dict_cache_tensor_indices_are_updated_in_place():
    ref = {"k": torch.zeros(1, 96, 1, 16), "v": torch.zeros(1, 96, 1, 16),
           "global_end_index": torch.tensor(0), "local_end_index": 0}
    q = torch.randn(1, 32, 1, 16)
    streaming_self_attention(q, q, q, ref, 0, attention_config=SDPA)
    streaming_self_attention(q, q, q, ref, 32, attention_config=SDPA)
    assert int(ref["global_end_index"]) == 64 and ref["local_end_index"] == 64
