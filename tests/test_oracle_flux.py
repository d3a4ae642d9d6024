"""Pins of the oracle's FLUX blocks (oracle/flux.py) at tiny width, CPU only.

Invariants that reduce the blocks to something computed another way: zero gates make a block
the identity; unit gates with zero shift/scale make it a plain pre-LN transformer block, built
here from torch's own SDPA / layer_norm / gelu; the single block's proj_out over the column
halves equals the one fused linear (tests/unit/quant/test_fake_linear.py:131-143).
"""

import math

import torch
import torch.nn.functional as F

from oracle import flux as oflux
from oracle import ops

SHAPE = oflux.FluxShape(hidden=64, heads=2, head_dim=32, n_double=1, n_single=1, in_channels=16,
                        out_channels=16, txt_dim=24, pooled_dim=12, axes=(8, 12, 12))


def _inputs(st=6, hw=(2, 3)):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, hw[0] * hw[1], 64, generator=g)
    c = torch.randn(1, st, 64, generator=g)
    t = torch.randn(1, 64, generator=g)
    cos, sin = ops.flux_pos_embed(ops.flux_ids(st, *hw), SHAPE.axes)
    return x, c, t, cos, sin


def _set_mod(w, name, n_chunks, gate_idx, gate_value):
    w[f"{name}.weight"].zero_()
    b = torch.zeros(n_chunks * 64)
    for gi in gate_idx:
        b[gi * 64:(gi + 1) * 64] = gate_value
    w[f"{name}.bias"] = b


def test_zero_gates_make_the_double_block_the_identity():
    w = oflux.double_block_weights(SHAPE, 1, 0)
    _set_mod(w, "norm1.linear", 6, (2, 5), 0.0)
    _set_mod(w, "norm1_context.linear", 6, (2, 5), 0.0)
    x, c, t, cos, sin = _inputs()
    c2, x2 = oflux.double_block(w, x, c, t, cos, sin, SHAPE)
    assert torch.equal(x2, x) and torch.equal(c2, c)


def _plain_joint_block(w, x, c, cos, sin):
    """Pre-LN joint transformer block with unit gates, from torch primitives."""
    def heads(t):
        return t.view(1, -1, 2, 32).transpose(1, 2)

    def rope(t):
        z = torch.view_as_complex(t.reshape(*t.shape[:-1], 16, 2).contiguous())
        ang = torch.atan2(sin[:, 0::2], cos[:, 0::2])
        return torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)).reshape(t.shape)

    def rms(t, wt):
        return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 1e-6) * wt

    ln = lambda t: F.layer_norm(t, (64,), eps=1e-6)  # noqa: E731
    lin = lambda t, n: F.linear(t, w[f"{n}.weight"], w[f"{n}.bias"])  # noqa: E731
    nx, nc = ln(x), ln(c)
    q = torch.cat([rms(heads(lin(nc, "attn.add_q_proj")), w["attn.norm_added_q.weight"]),
                   rms(heads(lin(nx, "attn.to_q")), w["attn.norm_q.weight"])], dim=2)
    k = torch.cat([rms(heads(lin(nc, "attn.add_k_proj")), w["attn.norm_added_k.weight"]),
                   rms(heads(lin(nx, "attn.to_k")), w["attn.norm_k.weight"])], dim=2)
    v = torch.cat([heads(lin(nc, "attn.add_v_proj")), heads(lin(nx, "attn.to_v"))], dim=2)
    o = F.scaled_dot_product_attention(rope(q), rope(k), v, scale=1 / math.sqrt(32))
    o = o.transpose(1, 2).reshape(1, -1, 64)
    st = c.shape[1]
    x = x + lin(o[:, st:], "attn.to_out.0")
    c = c + lin(o[:, :st], "attn.to_add_out")
    x = x + lin(F.gelu(lin(ln(x), "ff.net.0.proj"), approximate="tanh"), "ff.net.2")
    c = c + lin(F.gelu(lin(ln(c), "ff_context.net.0.proj"), approximate="tanh"), "ff_context.net.2")
    return c, x


def test_unit_gates_make_the_double_block_a_plain_transformer_block():
    w = oflux.double_block_weights(SHAPE, 2, 0)
    w["attn.norm_q.weight"] = torch.linspace(0.5, 1.5, 32)
    _set_mod(w, "norm1.linear", 6, (2, 5), 1.0)
    _set_mod(w, "norm1_context.linear", 6, (2, 5), 1.0)
    x, c, t, cos, sin = _inputs()
    c_ref, x_ref = _plain_joint_block(w, x, c, cos, sin)
    c2, x2 = oflux.double_block(w, x, c, t, cos, sin, SHAPE)
    assert torch.allclose(x2, x_ref, atol=1e-5) and torch.allclose(c2, c_ref, atol=1e-5)


def test_single_block_split_proj_out_equals_the_fused_linear():
    w = oflux.single_block_weights(SHAPE, 3, 0)
    x, c, t, cos, sin = _inputs()
    h = torch.cat([c, x], dim=1)
    out = oflux.single_block(w, h, t, cos, sin, SHAPE)
    # same block with proj_out as one linear over cat([attn, mlp])
    emb = F.linear(F.silu(t), w["norm.linear.weight"], w["norm.linear.bias"])
    shift, scale, gate = emb.chunk(3, dim=1)
    nh = ops.ada_modulate(h, shift, scale)
    mlp = F.gelu(F.linear(nh, w["proj_mlp.weight"], w["proj_mlp.bias"]), approximate="tanh")
    q, k, v = (F.linear(nh, w[f"attn.to_{n}.weight"], w[f"attn.to_{n}.bias"]).view(1, -1, 2, 32)
               .transpose(1, 2) for n in "qkv")
    q = ops.rms_norm_cpu_law(q, w["attn.norm_q.weight"], 1e-6)
    k = ops.rms_norm_cpu_law(k, w["attn.norm_k.weight"], 1e-6)
    q = ops.apply_rotary_emb_fp32(q, cos[None, None], sin[None, None])
    k = ops.apply_rotary_emb_fp32(k, cos[None, None], sin[None, None])
    o = F.scaled_dot_product_attention(q, k, v, scale=1 / math.sqrt(32)).transpose(1, 2).reshape(1, -1, 64)
    fused = F.linear(torch.cat([o, mlp], dim=-1), w["proj_out.weight"], w["proj_out.bias"])
    assert torch.allclose(out, h + gate[:, None] * fused, atol=1e-5)


def test_forward_shapes_and_weight_draws_are_seeded():
    shape = oflux.FluxShape(hidden=64, heads=2, head_dim=32, n_double=2, n_single=1,
                            in_channels=16, out_channels=16, txt_dim=24, pooled_dim=12,
                            axes=(8, 12, 12))
    inp = oflux.synthetic_inputs(shape, 5, (2, 3), 4)
    out = oflux.forward(shape, 5, inp["latents"], inp["text"], inp["pooled"], inp["timestep"],
                        inp["guidance"], (2, 3))
    assert out.shape == (1, 6, 16) and torch.isfinite(out).all()
    a = oflux.double_block_weights(shape, 5, 1)
    b = oflux.double_block_weights(shape, 5, 1)
    assert all(torch.equal(a[k], b[k]) for k in a)
    assert not torch.equal(a["ff.net.2.weight"], oflux.double_block_weights(shape, 5, 0)["ff.net.2.weight"])


# ------------------------------------------------------------------- against the reference model
def _reference_vectors():
    import json
    from pathlib import Path

    return json.loads((Path(__file__).parent / "golden" / "flux_reference_forward.json").read_text())


def test_forward_and_blocks_equal_the_reference_model():
    """The reference's own NeuronFluxTransformer2DModel (fp32, its CPU backend) ran on the same
    seeded weights and inputs (tests/golden/make_flux_golden.py): the oracle's forward, first
    double block (both streams) and first single block give the same values. They agreed to the
    last bit when the fixture was made; 1e-6 leaves room for another BLAS on another host."""
    from tests.golden.make_flux_golden import IMG_HW, SEED, SHAPE, TXT, decode, inputs

    g = _reference_vectors()
    assert g["shape"]["hidden"] == SHAPE.hidden and g["seed"] == SEED
    ref = {k: decode(v) for k, v in g["tensors"].items()}
    inp = inputs()
    f32 = torch.float32
    out = oflux.forward(SHAPE, SEED, inp["latents"], inp["text"], inp["pooled"], inp["timestep"],
                        inp["guidance"], IMG_HW, dtype=f32, model_dtype=f32)
    ew = oflux.embed_weights(SHAPE, SEED, dtype=f32)
    hidden = ops.linear(inp["latents"], ew["x_embedder.weight"], ew["x_embedder.bias"])
    context = ops.linear(inp["text"], ew["context_embedder.weight"], ew["context_embedder.bias"])
    temb = oflux.time_text_embed(ew, inp["timestep"] * 1000, inp["guidance"] * 1000,
                                 inp["pooled"], SHAPE)
    cos, sin = ops.flux_pos_embed(ops.flux_ids(TXT, *IMG_HW), SHAPE.axes)
    c0, h0 = oflux.double_block(oflux.double_block_weights(SHAPE, SEED, 0, dtype=f32),
                                hidden, context, temb, cos, sin, SHAPE)
    # the first single block's input: both double blocks, then [txt | img]
    c1, h1 = oflux.double_block(oflux.double_block_weights(SHAPE, SEED, 1, dtype=f32),
                                h0, c0, temb, cos, sin, SHAPE)
    s0 = oflux.single_block(oflux.single_block_weights(SHAPE, SEED, 0, dtype=f32),
                            torch.cat([c1, h1], dim=1), temb, cos, sin, SHAPE)
    for name, got in (("output", out), ("double0_context", c0), ("double0_hidden", h0),
                      ("single0", s0)):
        want = ref[name]
        assert got.shape == want.shape, name
        e = ((got - want).norm() / want.norm()).item()
        assert e < 1e-6, f"{name}: rel L2 {e:.3e}"


def test_a_planted_mistake_is_seen_by_the_reference_vectors():
    """The check is tight enough to fail a plausible slip: a wrong RoPE table (sin negated)."""
    from tests.golden.make_flux_golden import IMG_HW, SEED, SHAPE, TXT, decode, inputs

    want = decode(_reference_vectors()["tensors"]["double0_hidden"])
    inp = inputs()
    f32 = torch.float32
    ew = oflux.embed_weights(SHAPE, SEED, dtype=f32)
    hidden = ops.linear(inp["latents"], ew["x_embedder.weight"], ew["x_embedder.bias"])
    context = ops.linear(inp["text"], ew["context_embedder.weight"], ew["context_embedder.bias"])
    temb = oflux.time_text_embed(ew, inp["timestep"] * 1000, inp["guidance"] * 1000,
                                 inp["pooled"], SHAPE)
    cos, sin = ops.flux_pos_embed(ops.flux_ids(TXT, *IMG_HW), SHAPE.axes)
    _, h0 = oflux.double_block(oflux.double_block_weights(SHAPE, SEED, 0, dtype=f32),
                               hidden, context, temb, cos, -sin, SHAPE)
    assert ((h0 - want).norm() / want.norm()).item() > 1e-3
