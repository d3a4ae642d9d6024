"""Host side of the text encoders, on the CPU: the relative-position buckets the device bias is
built from, the config reader, the parameter layout, and the new kernels' refusals before any
device work."""

import dataclasses

import pytest
import torch

from difflet_amd import kernels
from difflet_amd.text import t5
from oracle import t5 as ot5

DEVICE_MSG = "rocm kernels take device tensors"


@pytest.mark.parametrize("sq,sk", [(1, 1), (7, 7), (150, 150), (512, 512), (3, 300)])
def test_host_buckets_equal_the_pinned_oracle_buckets(sq, sk):
    """buckets[j] is the bucket of relative position j - (sq - 1); the oracle's bucket function
    is bit-identical to transformers' (tests/test_oracle_t5.py)."""
    got = t5.relative_position_buckets(sq, sk, 32, 128)
    rel = torch.arange(-(sq - 1), sk)
    assert got.dtype == torch.int32 and got.shape == (sq + sk - 1,)
    assert torch.equal(got.long(), ot5.relative_position_bucket(rel, 32, 128))
    # the [sq, sk] table the device reads: entry (q, k) = buckets[k - q + sq - 1]
    q, k = torch.arange(sq)[:, None], torch.arange(sk)[None, :]
    assert torch.equal(got.long()[k - q + sq - 1], ot5.relative_position_bucket(k - q, 32, 128))


def test_param_layout_matches_the_hf_keys():
    for cfg, shape in ((t5.T5_XXL, ot5.T5_XXL), (t5.UMT5_XXL, ot5.UMT5_XXL)):
        assert t5.param_shapes(cfg) == dict(ot5.param_shapes(shape))
    assert sum("relative_attention_bias" in k for k in t5.param_shapes(t5.T5_XXL)) == 1
    assert sum("relative_attention_bias" in k for k in t5.param_shapes(t5.UMT5_XXL)) == 24


def test_config_from_hf_dict():
    raw = {"vocab_size": 256384, "d_model": 4096, "d_kv": 64, "d_ff": 10240, "num_heads": 64,
           "num_layers": 24, "relative_attention_num_buckets": 32,
           "relative_attention_max_distance": 128, "layer_norm_epsilon": 1e-6,
           "feed_forward_proj": "gated-gelu", "dense_act_fn": "gelu_new", "model_type": "umt5"}
    assert t5.T5Config.from_hf_dict(raw, umt5=True) == t5.UMT5_XXL
    small = dict(raw, vocab_size=32128)
    assert t5.T5Config.from_hf_dict(small, umt5=False) == t5.T5_XXL
    with pytest.raises(NotImplementedError):
        t5.T5Config.from_hf_dict(dict(raw, feed_forward_proj="relu"), umt5=True)


def test_encoder_refuses_unsupported_dtypes_and_widths():
    with pytest.raises(NotImplementedError):
        t5.T5Encoder(t5.T5_XXL, lambda n: None, dtype=torch.float16, device="cpu")
    with pytest.raises(NotImplementedError):
        t5.T5Encoder(dataclasses.replace(t5.T5_XXL, d_kv=80), lambda n: None, device="cpu")
    with pytest.raises(NotImplementedError):
        t5.T5Encoder(dataclasses.replace(t5.T5_XXL, d_ff=1000), lambda n: None, device="cpu")


def test_kernel_wrappers_refuse_before_device_work():
    f = torch.zeros
    with pytest.raises(ValueError, match=DEVICE_MSG):
        kernels.gemm_f32(f(4, 8), f(12, 8))
    with pytest.raises(ValueError, match="multiples of 4"):
        kernels.gemm_f32(f(4, 6), f(12, 6))
    with pytest.raises(ValueError, match="do not chain"):
        kernels.gemm_f32(f(4, 8), f(12, 12))
    with pytest.raises(ValueError, match="bias"):
        kernels.gemm_f32(f(4, 8), f(12, 8), f(8))
    with pytest.raises(ValueError, match="residual"):
        kernels.gemm_f32(f(4, 8), f(12, 8), residual=f(4, 8))
    with pytest.raises(TypeError):
        kernels.gemm_f32(f(4, 8, dtype=torch.bfloat16), f(12, 8))
    with pytest.raises(ValueError, match="gated_gelu"):
        kernels.gated_gelu(f(4, 15), 8)
    with pytest.raises(ValueError, match=DEVICE_MSG):
        kernels.gated_gelu(f(4, 16), 8)
    with pytest.raises(TypeError):
        kernels.embedding(torch.zeros(3, dtype=torch.int32), f(10, 8))
    with pytest.raises(IndexError):
        kernels.embedding(torch.tensor([10]), f(10, 8))
    with pytest.raises(ValueError, match=DEVICE_MSG):
        kernels.embedding(torch.tensor([9]), f(10, 8))
    b = t5.relative_position_buckets(5, 5, 32, 128)
    with pytest.raises(ValueError, match="buckets"):
        kernels.relative_bias(b[:-1], f(32, 4), batch=1, seq_q=5, seq_k=5)
    with pytest.raises(ValueError, match="key_keep"):
        kernels.relative_bias(b, f(32, 4), batch=2, seq_q=5, seq_k=5,
                              key_keep=torch.ones(1, 5, dtype=torch.bool))
    with pytest.raises(ValueError, match=DEVICE_MSG):
        kernels.relative_bias(b, f(32, 4), batch=1, seq_q=5, seq_k=5)
