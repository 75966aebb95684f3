"""torch.ops.telefuser_amd mirrors the op schemas of tf-kernel's SageAttention extension
(tf-kernel/csrc/common_extension.cc:168-260): same op names, argument names and order, in-place outputs.
Registration needs no GPU (the library loads on first call)."""

import torch

# argument names of the reference schemas (common_extension.cc), in order
REFERENCE_ARGS = {
    "quant_per_block_int8_cuda_with_sm_scale": ["input", "output", "scale", "sm_scale", "block_size", "tensor_layout"],
    "quant_per_block_int8_cuda": ["input", "output", "scale", "block_size", "tensor_layout"],
    "quant_per_block_int8_fuse_sub_mean_cuda": ["input", "mean", "output", "scale", "block_size", "tensor_layout"],
    "quant_per_warp_int8_cuda": ["input", "output", "scale", "block_size", "warp_block_size", "tensor_layout"],
    "qk_int8_sv_f8_accum_f32_fuse_v_scale_attn": ["query", "key", "value", "output", "query_scale", "key_scale",
                                                  "value_scale", "tensor_layout", "is_causal", "qk_quant_gran",
                                                  "sm_scale", "return_lse"],
    "qk_int8_sv_f8_accum_f32_fuse_v_scale_fuse_v_mean_attn": ["query", "key", "value", "output", "query_scale",
                                                              "key_scale", "value_scale", "value_mean",
                                                              "tensor_layout", "is_causal", "qk_quant_gran",
                                                              "sm_scale", "return_lse"],
    "qk_int8_sv_f16_accum_f32_attn": ["query", "key", "value", "output", "query_scale", "key_scale", "tensor_layout",
                                      "is_causal", "qk_quant_gran", "sm_scale", "return_lse"],
}
MUTATED = {"output", "scale"}


def test_ops_registered_with_reference_schemas():
    from telefuser_amd import ops

    for name in ops.OPS:
        assert hasattr(torch.ops.telefuser_amd, name), name
    for name, args in REFERENCE_ARGS.items():
        schema = getattr(torch.ops.telefuser_amd, name).default._schema
        got = [a.name for a in schema.arguments]
        assert got == args, f"{name}: {got}"
        for a in schema.arguments:
            written = a.alias_info is not None and a.alias_info.is_write
            assert written == (a.name in MUTATED), f"{name}.{a.name}"
        returns_tensor = len(schema.returns) == 1
        assert returns_tensor == name.startswith("qk_"), name
