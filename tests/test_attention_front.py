"""Host logic of the attention() front door (mirrors telefuser/ops/attention/attention_impl.py):
dispatch of the SAGE implementations to the drop-in module, layout handling, SDPA path and fallback.
Runs on the CPU with a recording stand-in for the Sage module (as the reference's
tests/unit/ops/test_attention_backends.py mocks its imports)."""

import types

import pytest
import torch

from telefuser_amd import attention as A


class _Recorder:
    def __init__(self):
        self.calls = []

    def _fn(self, name):
        def f(q, k, v, **kw):
            self.calls.append((name, q.shape, kw))
            out = q.clone()
            return (out, torch.zeros(1)) if kw.get("return_lse") else out
        return f


@pytest.fixture
def fake_sage(monkeypatch):
    rec = _Recorder()
    mod = types.SimpleNamespace(
        sageattn_qk_int8_pv_fp8_cuda=rec._fn("fp8"),
        sageattn_qk_int8_pv_fp16_cuda=rec._fn("fp16"),
        sageattn_qk_int8_pv_fp8_cuda_sm90=rec._fn("sm90"),
    )
    monkeypatch.setattr(A, "sageattention", mod)
    monkeypatch.setattr(A, "SAGE_ATTN_AVAILABLE", True)
    return rec


def test_sage_dispatch_keeps_bsnd_and_kwargs(fake_sage):
    q = torch.randn(1, 10, 2, 128)
    cfg = A.AttentionConfig(attn_impl=A.AttnImplType.SAGE_ATTN_2_8_8, scale=0.1)
    out = A.attention(q, q, q, attention_config=cfg, kv_valid_len=[7])
    name, shape, kw = fake_sage.calls[-1]
    assert name == "fp8" and shape == (1, 10, 2, 128)
    assert kw["tensor_layout"] == "NHD" and kw["sm_scale"] == 0.1 and kw["pv_accum_dtype"] == "fp32+fp32"
    assert kw["kv_valid_len"] == [7] and out.shape == q.shape


def test_sage_bnsd_input_is_converted(fake_sage):
    q = torch.randn(1, 2, 10, 128)  # BNSD
    out = A.attention(q, q, q, attn_impl=A.AttnImplType.SAGE_ATTN_2_8_16, input_layout="BNSD",
                      output_layout="BNSD")
    name, shape, kw = fake_sage.calls[-1]
    assert name == "fp16" and shape == (1, 10, 2, 128) and kw["tensor_layout"] == "NHD"
    assert kw["pv_accum_dtype"] == "fp32"
    assert out.shape == (1, 2, 10, 128)
    assert torch.equal(out, q)  # the stand-in returns q: round trip through both transposes


def test_return_lse_and_sm90(fake_sage):
    q = torch.randn(1, 4, 1, 128)
    out, lse = A.attention(q, q, q, attn_impl=A.AttnImplType.SAGE_ATTN_2_8_8_SM90, return_lse=True)
    assert fake_sage.calls[-1][0] == "sm90" and fake_sage.calls[-1][2]["return_lse"]
    assert A.supports_return_lse("SAGE_ATTN_2_8_8")


def test_sdpa_path_and_fallback_match_torch():
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 16, 3, 32) for _ in range(3))
    want = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True).transpose(1, 2)
    got = A.attention(q, k, v, attn_impl=A.AttnImplType.TORCH_SDPA, is_causal=True)
    assert torch.allclose(got, want, atol=1e-6)
    # an implementation this package does not provide falls back to SDPA
    got2 = A.attention(q, k, v, attn_impl=A.AttnImplType.FLASH_ATTN_3, is_causal=True)
    assert torch.allclose(got2, want, atol=1e-6)


def test_sage_impls_do_not_forward_is_causal(fake_sage):
    """The reference's SAGE branch calls the sage functions without is_causal (attention_impl.py:249-283),
    so a causal request through attention() yields the non-causal SAGE result; the front door matches."""
    q = torch.randn(1, 8, 2, 128)
    for impl in (A.AttnImplType.SAGE_ATTN_2_8_8, A.AttnImplType.SAGE_ATTN_2_8_16, A.AttnImplType.SAGE_ATTN_2_8_8_SM90):
        A.attention(q, q, q, attn_impl=impl, is_causal=True)
        assert "is_causal" not in fake_sage.calls[-1][2]
    A.attention(q, q, q, attention_config=A.AttentionConfig(attn_impl=A.AttnImplType.SAGE_ATTN_2_8_8, is_causal=True))
    assert "is_causal" not in fake_sage.calls[-1][2]
