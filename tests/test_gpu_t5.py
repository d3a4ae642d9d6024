"""The T5 / UMT5 text encoders on the HIP path against the fp32 oracle (oracle/t5.py, itself
bit-identical to transformers' encoders): the fp32 kernels and model within fp32 summation
order (rel L2 <= 1e-5), the bf16 ones against the oracle with the device's bf16 rounding points
(rel L2 <= 1e-2); the pieces (fp32 GEMM, gated GELU, embedding rows, relative bias) alone; the
full T5-XXL stack (24 blocks at 512 tokens) through properties."""

import dataclasses

import pytest
import torch

from difflet_amd import kernels
from difflet_amd.text.t5 import T5_XXL, T5Config, T5Encoder, random_param_source
from oracle import t5 as ot5

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _cfg(shape: ot5.T5Shape) -> T5Config:
    return T5Config(vocab_size=shape.vocab, d_model=shape.d_model, d_kv=shape.d_kv,
                    d_ff=shape.d_ff, num_heads=shape.heads, num_layers=shape.layers,
                    relative_attention_num_buckets=shape.buckets,
                    relative_attention_max_distance=shape.max_distance,
                    layer_norm_epsilon=shape.eps, per_layer_bias=shape.per_layer_bias)


# ----------------------------------------------------------------------------- kernels
@pytest.mark.parametrize("m,n,k", [(1, 4, 4), (77, 100, 60), (300, 520, 384), (512, 4096, 4096),
                                   (130, 4096, 10240)])
def test_gemm_f32_matches_fp32(gpu, m, n, k):
    print(f"gemm_f32 m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    a, w = torch.randn(m, k, generator=g), torch.randn(n, k, generator=g) / k ** 0.5
    bias, res = torch.randn(n, generator=g), torch.randn(m, n, generator=g)
    ref = a.double() @ w.double().T
    out = kernels.gemm_f32(a.to(gpu), w.to(gpu))
    assert rel_l2(out, ref) < 1e-5
    c = res.to(gpu)
    kernels.gemm_f32(a.to(gpu), w.to(gpu), bias.to(gpu), residual=c, out=c)  # residual aliases C
    assert rel_l2(c, res.double() + ref + bias.double()) < 1e-5


def test_gemm_f32_strided_views_and_refusals(gpu):
    g = torch.Generator().manual_seed(9)
    big = torch.randn(200, 256, generator=g)
    w = torch.randn(64, 128, generator=g)
    out = kernels.gemm_f32(big[:, 64:192].to(gpu), w.to(gpu))  # lda 256
    assert rel_l2(out, big[:, 64:192].double() @ w.double().T) < 1e-5
    with pytest.raises(ValueError, match="multiples of 4"):
        kernels.gemm_f32(torch.zeros(4, 6, device=gpu), torch.zeros(4, 6, device=gpu))
    with pytest.raises(TypeError):
        kernels.gemm_f32(torch.zeros(4, 8, device=gpu, dtype=torch.bfloat16),
                         torch.zeros(4, 8, device=gpu))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_gelu(gpu, dtype):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(133, 2 * 520, generator=g) * 3).to(dtype)
    ref = ot5.gelu_new(x[:, :520].float()) * x[:, 520:].float()
    out = kernels.gated_gelu(x.to(gpu), 520)
    assert out.dtype == dtype
    assert rel_l2(out, ref) < (2e-6 if dtype == torch.float32 else 4e-3)


def test_embedding_rows_and_refusals(gpu):
    g = torch.Generator().manual_seed(4)
    for dt in (torch.bfloat16, torch.float32):
        table = torch.randn(1000, 64, generator=g).to(dt)
        ids = torch.randint(0, 1000, (3, 77), generator=g)
        out = kernels.embedding(ids.to(gpu), table.to(gpu))
        assert torch.equal(out.cpu(), table[ids])
    with pytest.raises(IndexError):
        kernels.embedding(torch.tensor([[0, 1000]], device=gpu), table.to(gpu))
    with pytest.raises(IndexError):
        kernels.embedding(torch.tensor([[-1]], device=gpu), table.to(gpu))


@pytest.mark.parametrize("s", [1, 77, 512])
def test_relative_bias_equals_the_oracle_bias(gpu, s):
    from difflet_amd.text.t5 import relative_position_buckets

    g = torch.Generator().manual_seed(s)
    shape = ot5.T5Shape(heads=6)
    table = torch.randn(32, 6, generator=g).bfloat16()
    buckets = relative_position_buckets(s, s, 32, 128)
    out = kernels.relative_bias(buckets.to(gpu), table.to(gpu), batch=1, seq_q=s, seq_k=s)
    ref = ot5.position_bias(table.float(), s, s, shape)
    assert torch.equal(out.cpu(), ref)
    keep = torch.rand(2, s, generator=g) > 0.3
    out = kernels.relative_bias(buckets.to(gpu), table.float().to(gpu), batch=2, seq_q=s, seq_k=s,
                                key_keep=keep.to(gpu))
    want = ref.expand(2, -1, -1, -1).clone()
    want.masked_fill_(~keep[:, None, None, :], torch.finfo(torch.float32).min)
    assert torch.equal(out.cpu(), want)


def test_additive_lowest_float_mask_keeps_fully_masked_rows_finite(gpu):
    """A row whose every key carries finfo.min averages v (the reference's scores + mask stays
    finite in fp32), on the MFMA kernels (bf16, head_dim 64 and 128) and the fp32 kernel."""
    g = torch.Generator().manual_seed(12)
    for dt, d in ((torch.bfloat16, 64), (torch.bfloat16, 128), (torch.float32, 64)):
        q, k, v = (torch.randn(1, 2, 70, d, generator=g).to(dt) for _ in range(3))
        mask = torch.zeros(1, 2, 70, 70)
        mask[0, 1, 5] = torch.finfo(torch.float32).min
        mask[0, 0, :, 30:] = torch.finfo(torch.float32).min
        ref = ot5_attention(q, k, v, mask)
        out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=1.0,
                                attention_mask=mask.to(gpu))
        assert torch.isfinite(out.float()).all()
        assert rel_l2(out, ref) < (2e-5 if dt == torch.float32 else 1e-2)
        assert rel_l2(out[0, 1, 5], v[0, 1].float().mean(0)) < (2e-5 if dt == torch.float32 else 1e-2)


def ot5_attention(q, k, v, mask):
    from oracle import ops

    return ops.attention(q.float(), k.float(), v.float(), scale=1.0, attention_mask=mask)


# ----------------------------------------------------------------------------- encoders
SMALL = ot5.T5Shape(vocab=500, d_model=256, d_kv=64, d_ff=512, heads=4, layers=3)
SMALL_UMT5 = dataclasses.replace(SMALL, per_layer_bias=True)


@pytest.mark.parametrize("shape", [SMALL, SMALL_UMT5], ids=["t5", "umt5"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_encoder_matches_oracle(gpu, shape, dtype, parity):
    print(f"encoder {'umt5' if shape.per_layer_bias else 't5'} {dtype}", flush=True)
    w = ot5.weights(shape, 21, None if dtype == torch.float32 else dtype)
    enc = T5Encoder(_cfg(shape), lambda n: w[n], dtype=dtype, device=gpu)
    ids = torch.randint(0, shape.vocab, (2, 150), generator=torch.Generator().manual_seed(2))
    store = None if dtype == torch.float32 else dtype
    ref = ot5.encode(w, shape, ids, store=store)
    out = enc(ids)
    torch.cuda.synchronize()
    assert out.dtype == dtype and tuple(out.shape) == (2, 150, shape.d_model)
    e = rel_l2(out, ref)
    print(f"  rel L2 {e:.3e}", flush=True)
    bound = 1e-5 if dtype == torch.float32 else 1e-2
    parity(f"{'UMT5' if shape.per_layer_bias else 'T5'} 3-block encoder {str(dtype)[6:]}, rel L2 "
           "vs oracle", e, bound)
    assert e < bound


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_umt5_padding_mask_matches_oracle(gpu, dtype, parity):
    """Two prompts, the second right-padded after 97 of 150 tokens, and an all-padding one."""
    w = ot5.weights(SMALL_UMT5, 22, None if dtype == torch.float32 else dtype)
    enc = T5Encoder(_cfg(SMALL_UMT5), lambda n: w[n], dtype=dtype, device=gpu)
    ids = torch.randint(0, SMALL_UMT5.vocab, (3, 150), generator=torch.Generator().manual_seed(3))
    mask = torch.ones(3, 150, dtype=torch.long)
    mask[1, 97:] = 0
    mask[2] = 0
    store = None if dtype == torch.float32 else dtype
    ref = ot5.encode(w, SMALL_UMT5, ids, attention_mask=mask, store=store)
    out = enc(ids, attention_mask=mask.to(gpu))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    e = rel_l2(out, ref)
    print(f"  masked rel L2 {e:.3e}", flush=True)
    bound = 1e-5 if dtype == torch.float32 else 1e-2
    parity(f"UMT5 padded prompts {str(dtype)[6:]}, rel L2 vs oracle", e, bound)
    assert e < bound
    with pytest.raises(ValueError, match="no attention mask"):
        T5Encoder(_cfg(SMALL), lambda n: ot5.weights(SMALL, 1)[n], device=gpu)(ids, mask)


def test_umt5_width_two_blocks_fp32_matches_oracle(gpu, parity):
    """Two UMT5-XXL blocks at their real width (4096, 64 heads, d_ff 10240) on 512 tokens, fp32
    (the vocabulary cut to 1000 rows: it is a gather, not a dimension of the math)."""
    shape = dataclasses.replace(ot5.UMT5_XXL, vocab=1000, layers=2)
    w = ot5.weights(shape, 23)
    enc = T5Encoder(_cfg(shape), lambda n: w[n], dtype=torch.float32, device=gpu)
    ids = torch.randint(0, 1000, (1, 512), generator=torch.Generator().manual_seed(5))
    mask = torch.ones(1, 512, dtype=torch.long)
    mask[0, 300:] = 0
    out = enc(ids, attention_mask=mask.to(gpu))
    ref = ot5.encode(w, shape, ids, attention_mask=mask)
    e = rel_l2(out, ref)
    print(f"  umt5 width 2 blocks rel L2 {e:.3e}", flush=True)
    parity("UMT5-XXL width, 2 blocks fp32, rel L2 vs oracle", e, 1e-5)
    assert e < 1e-5


def test_t5_xxl_full_stack_bf16_and_fp32(gpu):
    """FLUX's T5-XXL (24 blocks, 4096 wide, 512 tokens) with random weights: both dtypes finite
    and bit-identical on a rerun, the bf16 stack within 5e-2 of the fp32 one."""
    cfg = dataclasses.replace(T5_XXL, vocab_size=1000)
    ids = torch.randint(0, 1000, (1, 512), generator=torch.Generator().manual_seed(6)).to(gpu)
    outs = {}
    for dt in (torch.float32, torch.bfloat16):
        print(f"t5-xxl full stack {dt}", flush=True)
        enc = T5Encoder(cfg, random_param_source(cfg, 5, gpu, torch.float32), dtype=dt, device=gpu)
        a, b = enc(ids), enc(ids)
        torch.cuda.synchronize()
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a, b)
        outs[dt] = a.float().cpu()
        del enc
        torch.cuda.empty_cache()
    e = rel_l2(outs[torch.bfloat16], outs[torch.float32])
    print(f"  bf16 vs fp32 rel L2 {e:.3e}", flush=True)
    assert e < 5e-2
