"""The rocm backend's op surface on the CPU host: every module difflet.ops resolves exists and
exports the reference's names, argument validation raises the reference's exceptions before
any device work, and the quantization spec keeps the reference's serialisation rules."""

import importlib

import pytest
import torch

OPS_EXPORTS = {  # difflet/ops/__init__.py:3-69 (module, name)
    "linear": ["ColumnParallelLinear", "ParallelEmbedding", "RowParallelLinear"],
    "norm": ["LayerNorm", "RMSNorm", "CustomRMSNorm", "rms_norm_fp32"],
    "collectives": ["SPMDRank", "gather_tp_dim", "init_parallel_mesh", "get_cfg_group",
                    "get_cp_group", "get_cfg_rank_spmd", "get_cp_rank_spmd", "get_world_group",
                    "gather_from_tensor_model_parallel_region_with_dim", "reduce_tp",
                    "reduce_from_tensor_model_parallel_region", "scatter_tp_dim",
                    "scatter_to_tensor_model_parallel_region", "scatter_to_process_group_spmd",
                    "scatter_to_sequence_parallel_region", "gather_from_sequence_parallel_region",
                    "reduce_scatter_to_sequence_parallel_region", "get_tp_rank", "get_tp_size",
                    "get_tensor_model_parallel_rank", "get_tensor_model_parallel_size"],
    "attention": ["attention", "cross_attention", "ring_attention", "joint_ring_attention",
                  "ulysses_attention", "joint_ulysses_attention"],
    "embeddings": ["apply_rotary_emb", "apply_rotary_emb_fp32"],
    "markers": ["ModuleMarkerStartWrapper", "ModuleMarkerEndWrapper"],
    "mx": ["dequantize_mx", "linear_mx", "matmul_mx", "quantize_mx"],
    "platform": ["get_platform_target", "hardware"],
}


@pytest.mark.parametrize("module", sorted(OPS_EXPORTS))
def test_every_op_module_exists_and_exports_the_names(module):
    mod = importlib.import_module(f"difflet_amd.backends.rocm.ops_impl.{module}")
    for name in OPS_EXPORTS[module]:
        assert hasattr(mod, name), f"{module}.{name}"


def test_platform_enum_and_markers():
    from difflet_amd.backends.rocm.ops_impl import markers, platform

    assert platform.hardware.TRN1 and platform.get_platform_target() is platform.hardware.ROCM
    x = torch.ones(3)
    assert markers.ModuleMarkerStartWrapper()(x) is x
    assert markers.ModuleMarkerEndWrapper()(x, x) == (x, x)


def test_attention_validation_precedes_device_work():
    from difflet_amd.backends.rocm.ops_impl import attention as A

    q = torch.zeros(1, 4, 128)
    b = torch.zeros(1, 4, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="both"):
        A.attention(q, q, q, bound_min=b)
    with pytest.raises(ValueError, match="exclusive"):
        A.attention(q, q, q, bound_min=b, bound_max=b, attention_mask=torch.ones(4, 4, dtype=torch.bool))
    with pytest.raises(ValueError, match="device"):
        A.attention(q, q, q)


def test_mx_ops_refuse_like_the_cuda_backend():
    from difflet_amd.backends.rocm.ops_impl import mx

    for fn in (mx.quantize_mx, mx.dequantize_mx, mx.linear_mx, mx.matmul_mx):
        with pytest.raises(NotImplementedError):
            fn(torch.zeros(8, 8))


def test_collectives_are_identities_at_world_size_one():
    from difflet_amd.backends.rocm.ops_impl import collectives as C

    x = torch.arange(6.0)
    assert C.reduce_tp(x) is x and C.gather_tp_dim(x, dim=0) is x
    assert C.reduce_from_tensor_model_parallel_region(x) is x
    assert C.scatter_to_sequence_parallel_region(x, dim=0) is x
    assert C.get_world_group().size() == 1 and C.get_tp_size() == 1
    assert C.get_cfg_rank_spmd(3) == 0
    assert int(C.SPMDRank(1).get_rank()) == 0


def test_collectives_refuse_several_ranks(monkeypatch):
    from difflet_amd.backends.rocm.ops_impl import collectives as C

    monkeypatch.setenv("WORLD_SIZE", "2")
    with pytest.raises(NotImplementedError):
        C.reduce_tp(torch.zeros(2))


def test_linear_and_norm_modules_keep_the_reference_state_dicts():
    from difflet_amd.backends.rocm.ops_impl import linear, norm

    col = linear.ColumnParallelLinear(16, 8, bias=True, gather_output=False, reduce_dtype=torch.bfloat16)
    row = linear.RowParallelLinear(16, 8, bias=False, skip_bias_add=True, reduce_output=False)
    assert set(col.state_dict()) == {"weight", "bias"} and set(row.state_dict()) == {"weight"}
    assert col.weight.shape == (8, 16) and row.skip_bias_add and row.tensor_parallel_group is None
    assert set(norm.RMSNorm(32, eps=1e-6).state_dict()) == {"weight"}
    ln = norm.LayerNorm(32, elementwise_affine=False, eps=1e-6)
    assert ln.weight is None and ln.bias is None
    assert norm.CustomRMSNorm is norm.RMSNorm


def test_quant_spec_rules():
    from difflet_amd.quant import spec as S

    sp = S.RocmQuantSpec(targets=S.QWEN_IMAGE_TARGETS)
    assert sp.matches("transformer.transformer_blocks.3.attn.to_q")
    assert not sp.matches("transformer_blocks.3.attn.to_out.0")
    assert sp.unmatched_targets(["transformer_blocks.0.attn.to_q"]) == list(S.QWEN_IMAGE_TARGETS[1:])
    assert S.RocmQuantSpec.from_dict(sp.to_dict()) == sp
    assert sp.cache_fields()["quant"] == "mxfp8" and sp.cache_fields()["quant_compute"] == "rocm"
    fp8 = S.RocmQuantSpec(targets=S.FLUX_ALL_BLOCK_LINEARS, format="fp8_rowwise")
    assert fp8.cache_fields()["quant"] == "fp8_rowwise"
    with pytest.raises(ValueError):
        S.RocmQuantSpec(targets=("x",), compute="nki")
    with pytest.raises(ValueError):
        S.RocmQuantSpec(targets=("x",), tp_degree=2)


def test_quantize_module_refuses_dead_targets_and_swaps_in_place():
    from difflet_amd.backends.rocm.ops_impl import linear
    from difflet_amd.quant import linear as Q
    from difflet_amd.quant.spec import RocmQuantSpec

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.to_q = linear.ColumnParallelLinear(128, 128, device="meta", dtype=torch.bfloat16)
            self.to_out = torch.nn.ModuleList([linear.RowParallelLinear(128, 128, device="meta",
                                                                         dtype=torch.bfloat16)])

    m = torch.nn.Module()
    m.attn = Attn()
    with pytest.raises(ValueError, match="match no linear"):
        Q.quantize_module_(m, RocmQuantSpec(targets=(r"attn\.to_k",)))
    names = Q.quantize_module_(m, RocmQuantSpec(targets=(r"attn\.(to_q|to_out\.0)",),
                                                format="fp8_rowwise"))
    assert names == ["attn.to_q", "attn.to_out.0"]
    assert isinstance(m.attn.to_q, Q.FP8ColumnParallelLinear)
    assert isinstance(m.attn.to_out[0], Q.FP8RowParallelLinear)
    assert m.attn.to_q.weight.dtype == torch.float8_e4m3fn and m.attn.to_q.weight_scale.shape == (128,)
