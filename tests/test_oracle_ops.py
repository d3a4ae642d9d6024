"""Pins of the oracle's op restatements (oracle/ops.py), CPU only: literal known answers from
the reference's tests, closed forms, and library routines computed another way."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ops


def test_stride2_rope_known_answer():
    """tests/unit/ops/test_ops_public_api.py:98-117 (values written out)."""
    x = torch.tensor([[[[1.0, 2.0, 3.0, 4.0]]]])
    cos = torch.tensor([[[[10.0, 20.0, 30.0, 40.0]]]])
    sin = torch.tensor([[[[0.5, 0.25, 0.125, 0.0625]]]])
    out = ops.apply_rotary_emb(x, cos, sin)
    assert torch.equal(out, torch.tensor([[[[9.5, 20.25, 89.75, 120.1875]]]]))


def test_fp32_rope_is_complex_rotation():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 5, 8, generator=g)
    theta = torch.randn(5, 4, generator=g)
    cos = theta.cos().repeat_interleave(2, dim=-1)
    sin = theta.sin().repeat_interleave(2, dim=-1)
    out = ops.apply_rotary_emb_fp32(x, cos, sin)
    z = torch.view_as_complex(x.reshape(2, 3, 5, 4, 2).contiguous())
    ref = torch.view_as_real(z * torch.polar(torch.ones_like(theta), theta)).reshape(2, 3, 5, 8)
    assert torch.allclose(out, ref, atol=1e-6)


def test_rms_norm_fp32_law_bit_exact_and_library():
    """tests/unit/backends/test_rms_norm_fp32_op.py:14-30 (the law, bit for bit), and
    F.rms_norm within fp32 rounding."""
    g = torch.Generator().manual_seed(1)
    for dt in (torch.float32, torch.bfloat16):
        x = torch.randn(3, 7, 32, generator=g).to(dt)
        w = (torch.rand(32, generator=g) + 0.5).to(dt)
        sq = x.float().pow(2).sum(-1, keepdim=True)
        manual = (x.float() * torch.rsqrt(sq / 32 + 1e-6) * w.float()).to(dt)
        assert torch.equal(ops.rms_norm_fp32(x, w, 1e-6), manual)
    x = torch.randn(4, 64, generator=g)
    assert torch.allclose(ops.rms_norm_fp32(x, None, 1e-6), F.rms_norm(x, (64,), eps=1e-6),
                          atol=1e-6)


def test_rms_norm_cpu_law_on_constant_rows():
    x = torch.full((2, 16), -3.0)
    w = torch.arange(16, dtype=torch.float32)
    assert torch.allclose(ops.rms_norm_cpu_law(x, w, 0.0), -w)


def test_attention_closed_forms():
    g = torch.Generator().manual_seed(2)
    v = torch.randn(2, 9, 8, generator=g)
    k = torch.randn(2, 9, 8, generator=g)
    q = torch.zeros(2, 5, 8)
    out = ops.attention(q, k, v, scale=0.3)  # equal scores: uniform weights
    assert torch.allclose(out, v.mean(dim=1, keepdim=True).expand(2, 5, 8), atol=1e-6)
    q = torch.randn(2, 5, 8, generator=g)
    ref = F.scaled_dot_product_attention(q, k, v, scale=0.3)
    assert torch.allclose(ops.attention(q, k, v, scale=0.3), ref, atol=1e-5)
    assert torch.allclose(ops.attention(q, k, v), F.scaled_dot_product_attention(q, k, v, scale=1.0),
                          atol=1e-5)  # scale=None means 1.0
    causal = ops.attention(q[:, :1], k[:, :1], v[:, :1], causal=True)
    assert torch.allclose(causal, v[:, :1], atol=1e-6)


def test_attention_bounds_equal_mask_and_empty_rows_average():
    """tests/unit/backends/test_cpu_ops_impl.py:492-517."""
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 6, 4, generator=g) for _ in range(3))
    bmin = torch.tensor([0, 1, 2, 0, 3, 5]).view(1, 6, 1).expand(2, 6, 1)
    bmax = torch.tensor([6, 4, 2, 1, 6, 6]).view(1, 6, 1).expand(2, 6, 1)
    key = torch.arange(6).view(1, 1, 6)
    mask = (key >= bmin) & (key < bmax)
    a = ops.attention(q, k, v, scale=0.5, bound_min=bmin, bound_max=bmax)
    b = ops.attention(q, k, v, scale=0.5, attention_mask=mask)
    assert torch.equal(a, b)
    assert torch.allclose(a[:, 2], v.mean(dim=1), atol=1e-6)  # row 2: empty window
    with pytest.raises(ValueError):
        ops.attention(q, k, v, bound_min=bmin)
    with pytest.raises(ValueError):
        ops.attention(q, k, v, bound_min=bmin, bound_max=bmax, attention_mask=mask)


def test_layer_norm_modulation_invariants():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 5, 64, generator=g) * 3 + 1
    y = ops.ada_modulate(x, torch.zeros(2, 64), torch.zeros(2, 64))
    assert torch.allclose(y.mean(-1), torch.zeros(2, 5), atol=1e-5)
    assert torch.allclose(y.var(-1, unbiased=False), torch.ones(2, 5), atol=1e-3)
    sh, sc = torch.randn(2, 64, generator=g), torch.randn(2, 64, generator=g)
    assert torch.allclose(ops.ada_modulate(x, sh, sc), y * (1 + sc[:, None]) + sh[:, None],
                          atol=1e-5)


def test_gelu_tanh_closed_form():
    for v in (-5.0, -1.3, -0.2, 0.0, 0.7, 2.5, 9.0):
        ref = 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
        assert abs(ops.gelu_tanh(torch.tensor([v]))[0].item() - ref) < 1e-6


def test_timestep_embedding_closed_form():
    t = torch.tensor([0.0, 250.0])
    e = ops.timestep_embedding(t, 8, flip_sin_to_cos=True, downscale_freq_shift=0)
    assert torch.allclose(e[0], torch.tensor([1.0] * 4 + [0.0] * 4))
    freqs = [math.exp(-math.log(10000) * i / 4) for i in range(4)]
    ref = [math.cos(250 * f) for f in freqs] + [math.sin(250 * f) for f in freqs]
    assert torch.allclose(e[1], torch.tensor(ref), atol=1e-4)


def test_flux_rope_tables_closed_form():
    ids = ops.flux_ids(2, 3, 4)
    assert ids.shape == (14, 3) and ids[:2].abs().sum() == 0
    assert ids[2 + 1 * 4 + 3].tolist() == [0.0, 1.0, 3.0]
    cos, sin = ops.flux_pos_embed(ids)
    assert cos.shape == (14, 128)
    row = 2 + 2 * 4 + 1  # patch (2, 1)
    for c, (axis, off, d) in enumerate([(0, 0, 16), (1, 16, 56), (2, 72, 56)]):
        for i in range(0, d, 2):
            ang = ids[row, axis].item() * 10000.0 ** (-i / d)
            assert abs(cos[row, off + i].item() - math.cos(ang)) < 1e-6
            assert abs(sin[row, off + i + 1].item() - math.sin(ang)) < 1e-6


def test_attention_equals_the_reference_cpu_op_on_every_form():
    """The reference CPU backend's attention op ran on the same seeded inputs
    (tests/golden/make_attention_golden.py): plain, scale None, causal, bool mask with a fully
    masked row, additive mask, per-query bounds on the (B*H, S, D) layout, in fp32 and bf16. The
    oracle matched it to the last bit when the fixture was made."""
    import json
    from pathlib import Path

    from tests.golden.make_attention_golden import cases, decode

    g = json.loads((Path(__file__).parent / "golden" / "attention_reference.json").read_text())
    for dtype, tol in ((torch.float32, 1e-6), (torch.bfloat16, 1e-3)):
        for name, ((q, k, v), kw) in cases(dtype).items():
            want = decode(g[f"{name}.{str(dtype).removeprefix('torch.')}"])
            got = ops.attention(q, k, v, **kw)
            assert got.dtype == dtype and tuple(got.shape) == tuple(want.shape), name
            e = ((got.float() - want).norm() / want.norm()).item()
            assert e < tol, f"{name} {dtype}: rel L2 {e:.3e}"
