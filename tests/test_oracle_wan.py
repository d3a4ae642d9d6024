"""The Wan oracle and the Wan step's host-side layout helpers."""

import torch

from oracle import ops
from oracle import wan as owan

SMALL = owan.WanShape(hidden=256, heads=2, head_dim=128, ffn=384, n_blocks=1, text_dim=64)


def test_rope_tables_axes_and_closed_form():
    assert owan.rope_dims(128) == (44, 42, 42)
    cos, sin = owan.rope_tables((2, 3, 4))
    assert cos.shape == (24, 128)
    # token (f, y, x) = (1, 2, 3): angles f * w_t, y * w_h, x * w_w with w = theta^(-2i/dim)
    r = 1 * 12 + 2 * 4 + 3
    for (lo, dim, pos) in ((0, 44, 1), (44, 42, 2), (86, 42, 3)):
        w = 1.0 / 10000.0 ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim)
        assert torch.allclose(cos[r, lo:lo + dim:2].double(), torch.cos(pos * w), atol=1e-6)
        assert torch.allclose(sin[r, lo + 1:lo + dim:2].double(), torch.sin(pos * w), atol=1e-6)


def test_device_rope_tables_equal_the_oracle():
    from difflet_amd.dit.rope import wan_rope_tables

    for grid in ((21, 30, 52), (2, 4, 6)):
        c0, s0 = owan.rope_tables(grid)
        c1, s1 = wan_rope_tables(grid, device="cpu")
        assert torch.equal(c0, c1) and torch.equal(s0, s1)


def test_patchify_linear_is_the_patch_conv3d_and_unpatchify_inverts():
    from difflet_amd.dit.wan import patchify, unpatchify

    g = torch.Generator().manual_seed(0)
    lat = torch.randn(1, 16, 3, 8, 10, generator=g)
    w, b = torch.randn(32, 16, 1, 2, 2, generator=g), torch.randn(32, generator=g)
    conv = torch.nn.functional.conv3d(lat, w, b, stride=(1, 2, 2)).flatten(2).transpose(1, 2)[0]
    lin = patchify(lat[0], (1, 2, 2)) @ w.reshape(32, -1).T + b
    assert torch.allclose(conv, lin, atol=1e-5)
    # unpatchify of per-token features in (kt, kh, kw, c) order against the reference's reshape
    grid = (3, 4, 5)
    y = torch.randn(60, 4 * 16, generator=g)
    ref = y.reshape(1, *grid, 1, 2, 2, -1).permute(0, 7, 1, 4, 2, 5, 3, 6)
    ref = ref.flatten(6, 7).flatten(4, 5).flatten(2, 3)
    assert torch.equal(unpatchify(y, grid, (1, 2, 2)), ref)


def _block_inputs(seed=0, s=6, st=3):
    g = torch.Generator().manual_seed(seed)
    d = SMALL.hidden
    return (torch.randn(1, s, d, generator=g), torch.randn(1, st, d, generator=g),
            torch.randn(1, 6, d, generator=g) * 0.1)


def test_zero_gates_and_zero_cross_output_make_the_block_the_identity():
    w = owan.block_weights(SMALL, 1, 0, dtype=torch.float32)
    hidden, text, tproj = _block_inputs()
    w["scale_shift_table"][:, 2] = -tproj[:, 2]  # gate = table + proj = 0
    w["scale_shift_table"][:, 5] = -tproj[:, 5]  # c_gate = 0
    w["attn2.to_out.0.weight"].zero_()
    w["attn2.to_out.0.bias"].zero_()
    cos, sin = owan.rope_tables((1, 2, 3), SMALL)
    assert torch.equal(owan.block(w, hidden, text, tproj, cos, sin, SMALL), hidden)


def test_cross_attention_with_one_text_token_adds_its_projected_value():
    """One text key: softmax is 1, the cross-attention output is to_out(to_v(text)) for every
    query."""
    w = owan.block_weights(SMALL, 2, 0, dtype=torch.float32)
    hidden, text, tproj = _block_inputs(1, st=1)
    w["scale_shift_table"][:, 2] = -tproj[:, 2]
    w["scale_shift_table"][:, 5] = -tproj[:, 5]
    cos, sin = owan.rope_tables((1, 2, 3), SMALL)
    out = owan.block(w, hidden, text, tproj, cos, sin, SMALL)
    L = ops.linear
    v = L(text, w["attn2.to_v.weight"], w["attn2.to_v.bias"])
    ref = hidden + L(v, w["attn2.to_out.0.weight"], w["attn2.to_out.0.bias"])
    assert torch.allclose(out, ref, atol=1e-5)


# ------------------------------------------------ unit gates: a plain transformer block
def _unit_gate_case(seed=21, s=6, st=4):
    """Zero shift / scale and unit gates (table + proj), random affine norm2 and random q/k
    RMSNorm weights over the whole width."""
    w = owan.block_weights(SMALL, seed, 0, dtype=torch.float32)
    hidden, text, tproj = _block_inputs(seed, s=s, st=st)
    table = torch.zeros(1, 6, SMALL.hidden)
    table[:, 2] = 1.0
    table[:, 5] = 1.0
    w["scale_shift_table"] = table - tproj
    g = torch.Generator().manual_seed(seed)
    for a in ("attn1", "attn2"):
        for n in ("norm_q", "norm_k"):
            w[f"{a}.{n}.weight"] = 0.5 + torch.rand(SMALL.hidden, generator=g)
    w["norm2.weight"] = 0.5 + torch.rand(SMALL.hidden, generator=g)
    w["norm2.bias"] = 0.1 * torch.randn(SMALL.hidden, generator=g)
    cos, sin = owan.rope_tables((1, 2, 3), SMALL)
    return w, hidden, text, tproj, cos, sin


def _plain_wan_block(w, x, text, cos, sin):
    """Wan's block with unit gates and no modulation, from torch primitives: F.rms_norm over the
    whole width (across heads), RoPE as complex multiplication of consecutive pairs,
    F.scaled_dot_product_attention, affine F.layer_norm before the cross-attention, then
    LayerNorm and a GELU(tanh) FFN (modeling_wan.py:564-578,720-763)."""
    import torch.nn.functional as F

    d = SMALL.hidden
    heads = lambda t: t.view(1, -1, 2, 128).transpose(1, 2)  # noqa: E731
    merge = lambda t: t.transpose(1, 2).reshape(1, -1, d)  # noqa: E731
    lin = lambda t, n: F.linear(t, w[f"{n}.weight"], w[f"{n}.bias"])  # noqa: E731
    rms = lambda t, n: F.rms_norm(t, (d,), w[f"{n}.weight"], 1e-6)  # noqa: E731
    ang = torch.atan2(sin[:, 1::2], cos[:, 0::2])

    def rope(t):  # [1, S, D] as heads
        h = heads(t)
        z = torch.view_as_complex(h.reshape(*h.shape[:-1], 64, 2).contiguous())
        return torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)).reshape(h.shape)

    n1 = F.layer_norm(x, (d,), eps=1e-6)
    q = rope(rms(lin(n1, "attn1.to_q"), "attn1.norm_q"))
    k = rope(rms(lin(n1, "attn1.to_k"), "attn1.norm_k"))
    x = x + lin(merge(F.scaled_dot_product_attention(q, k, heads(lin(n1, "attn1.to_v")))),
                "attn1.to_out.0")
    n2 = F.layer_norm(x, (d,), w["norm2.weight"], w["norm2.bias"], 1e-6)
    q = heads(rms(lin(n2, "attn2.to_q"), "attn2.norm_q"))
    k = heads(rms(lin(text, "attn2.to_k"), "attn2.norm_k"))
    x = x + lin(merge(F.scaled_dot_product_attention(q, k, heads(lin(text, "attn2.to_v")))),
                "attn2.to_out.0")
    ff = lin(F.gelu(lin(F.layer_norm(x, (d,), eps=1e-6), "ffn.net_in"), approximate="tanh"),
             "ffn.net_out")
    return x + ff


def test_unit_gates_make_the_block_a_plain_transformer_block():
    """Self-attention (across-heads RMSNorm, stride-2 RoPE), the affine norm2 and
    cross-attention, and the FFN, against torch's own primitives."""
    w, hidden, text, tproj, cos, sin = _unit_gate_case()
    ref = _plain_wan_block(w, hidden, text, cos, sin)
    out = owan.block(w, hidden, text, tproj, cos, sin, SMALL)
    assert torch.allclose(out, ref, atol=1e-5, rtol=1e-5)


def test_planted_exact_gelu_is_seen_by_the_plain_block(monkeypatch):
    w, hidden, text, tproj, cos, sin = _unit_gate_case()
    ref = _plain_wan_block(w, hidden, text, cos, sin)
    monkeypatch.setattr(ops, "gelu_tanh", lambda x: torch.nn.functional.gelu(x))
    assert not torch.allclose(owan.block(w, hidden, text, tproj, cos, sin, SMALL), ref,
                              atol=1e-5, rtol=1e-5)


def test_planted_per_head_rms_norm_is_seen_by_the_plain_block(monkeypatch):
    """An oracle that normalises q and k per head (FLUX's law) instead of across all heads
    fails the check."""
    w, hidden, text, tproj, cos, sin = _unit_gate_case()
    ref = _plain_wan_block(w, hidden, text, cos, sin)
    across = ops.rms_norm_fp32

    def per_head(x, weight, eps):
        h = x.unflatten(-1, (-1, 128))
        y = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
        return y.flatten(-2) * weight

    monkeypatch.setattr(ops, "rms_norm_fp32", per_head)
    assert not torch.allclose(owan.block(w, hidden, text, tproj, cos, sin, SMALL), ref, atol=1e-4)
    monkeypatch.setattr(ops, "rms_norm_fp32", across)
    assert torch.allclose(owan.block(w, hidden, text, tproj, cos, sin, SMALL), ref, atol=1e-5,
                          rtol=1e-5)


def test_planted_swapped_chunk_order_is_seen_by_the_plain_block():
    """timestep_proj with its gate and scale chunks exchanged (an oracle reading the six
    vectors in another order) fails the check."""
    w, hidden, text, tproj, cos, sin = _unit_gate_case()
    ref = _plain_wan_block(w, hidden, text, cos, sin)
    mods = w["scale_shift_table"] + tproj
    swapped = mods[:, [0, 2, 1, 3, 4, 5]] - w["scale_shift_table"]
    assert not torch.allclose(owan.block(w, hidden, text, swapped, cos, sin, SMALL), ref, atol=1e-3)


def test_planted_per_head_rope_table_offset_is_seen():
    """RoPE applied with the table of the wrong token (rows shifted by one) fails the check:
    the self-attention path is not left unpinned by the gates."""
    w, hidden, text, tproj, cos, sin = _unit_gate_case()
    ref = _plain_wan_block(w, hidden, text, cos, sin)
    out = owan.block(w, hidden, text, tproj, cos.roll(1, 0), sin.roll(1, 0), SMALL)
    assert not torch.allclose(out, ref, atol=1e-4)


# ------------------------------------- step level: conditioning and the final layer, pinned
# Reductions of the step-level functions to torch primitives and closed forms: identity
# linears make the time embedder silu(sinusoid) and the text projection GELU(tanh); distinct
# shift / scale vectors and an identity proj_out make the final layer one F.layer_norm
# expression. Each check is paired with a planted mistake that fails it.
COND = owan.WanShape(hidden=256, heads=2, head_dim=128, ffn=384, n_blocks=0, text_dim=256)
T_STEPS = torch.tensor([0.0, 999.7, 317.25])  # 999.7 is not a bf16 value (bf16 rounds it to 1000)


def _sinusoid64(t, dim=256):
    """get_timestep_embedding(t, 256, flip_sin_to_cos=True, downscale_freq_shift=0) as the
    reference parameterises it (modeling_wan.py:341-343), in float64: frequencies
    exp(-ln(10000) i / 128) for i < 128, cos half first."""
    import math

    import numpy as np

    half = dim // 2
    f = np.exp(-math.log(10000.0) * np.arange(half) / half)
    a = np.outer(np.asarray(t, dtype=np.float64), f)
    return torch.from_numpy(np.concatenate([np.cos(a), np.sin(a)], axis=1))


def _identity_condition(seed=3):
    d = COND.hidden
    ew = owan.embed_weights(COND, seed, dtype=torch.float32)
    p = "condition_embedder."
    eye = torch.eye(d)
    for n in ("time_embedder.linear_1", "time_embedder.linear_2", "text_embedder.linear_1",
              "text_embedder.linear_2"):
        ew[f"{p}{n}.weight"], ew[f"{p}{n}.bias"] = eye.clone(), torch.zeros(d)
    c = torch.tensor([0.5, -1.0, 2.0, 0.25, -0.75, 1.5])
    ew[p + "time_proj.weight"] = torch.cat([ci * eye for ci in c])
    ew[p + "time_proj.bias"] = torch.linspace(-1.0, 1.0, 6 * d)
    text = torch.randn(1, 5, d, generator=torch.Generator().manual_seed(seed)) * 1.5
    return ew, c, text


def _check_condition(ew, c, text, model_dtype=torch.float32):
    """True when condition() equals the closed forms: temb = silu(sinusoid(t)), timestep_proj
    chunk i = c_i silu(temb) + b_i, text = GELU_tanh(text)."""
    import torch.nn.functional as F

    d = COND.hidden
    temb, tproj, txt = owan.condition(ew, T_STEPS, text, model_dtype)
    tp = _sinusoid64(T_STEPS)
    if model_dtype == torch.float32:
        ref_temb, tol = F.silu(tp), 3e-4  # fp32 arguments up to 1000 rad: ~1e-4
    else:  # the sinusoid and temb rounded to the model dtype (two roundings: 2 ulp)
        ref_temb, tol = F.silu(tp.to(model_dtype).double()).to(model_dtype).double(), 8e-3
    ok = torch.allclose(temb.double(), ref_temb, atol=tol, rtol=0)
    b = ew["condition_embedder.time_proj.bias"].view(6, d).double()
    ref_proj = c.double()[:, None] * F.silu(ref_temb)[:, None, :] + b
    ok &= torch.allclose(tproj.double(), ref_proj, atol=3 * tol, rtol=2 * tol)
    ok &= torch.allclose(txt, F.gelu(text, approximate="tanh"), atol=1e-6, rtol=1e-6)
    return bool(ok)


def test_condition_reduces_to_silu_sinusoid_and_gelu_tanh():
    ew, c, text = _identity_condition()
    assert _check_condition(ew, c, text)
    assert _check_condition(ew, c, text, torch.bfloat16)
    # t = 0: the sinusoid is cos 0 = 1 on the first half and sin 0 = 0 on the second
    temb, _, _ = owan.condition(ew, torch.zeros(1), text)
    assert torch.allclose(temb[0, :128], torch.nn.functional.silu(torch.ones(128)))
    assert torch.equal(temb[0, 128:], torch.zeros(128))


def test_planted_exact_gelu_in_the_text_projection_is_seen(monkeypatch):
    ew, c, text = _identity_condition()
    monkeypatch.setattr(ops, "gelu_tanh", lambda x: torch.nn.functional.gelu(x))
    assert not _check_condition(ew, c, text)


def test_planted_sin_first_sinusoid_is_seen(monkeypatch):
    ew, c, text = _identity_condition()
    real = ops.timestep_embedding
    monkeypatch.setattr(ops, "timestep_embedding",
                        lambda t, dim, **kw: real(t, dim, **{**kw, "flip_sin_to_cos": False}))
    assert not _check_condition(ew, c, text)


def test_planted_timestep_cast_before_the_sinusoid_is_seen(monkeypatch):
    """Wan takes the sinusoid of the fp32 timestep and casts its output to the model dtype
    (modeling_wan.py:356-361); an oracle that casts t itself to bf16 first (FLUX's order)
    fails at t = 999.7."""
    ew, c, text = _identity_condition()
    real = ops.timestep_embedding
    monkeypatch.setattr(ops, "timestep_embedding",
                        lambda t, dim, **kw: real(t.to(torch.bfloat16).float(), dim, **kw))
    assert not _check_condition(ew, c, text, torch.bfloat16)


FINAL = owan.WanShape(hidden=64, heads=1, head_dim=64, ffn=128, n_blocks=0, text_dim=64)


def _final_case(seed=4):
    g = torch.Generator().manual_seed(seed)
    ew = owan.embed_weights(FINAL, seed, dtype=torch.float32)
    ew["proj_out.weight"], ew["proj_out.bias"] = torch.eye(64), torch.zeros(64)
    ew["scale_shift_table"] = torch.randn(1, 2, 64, generator=g)
    hidden = torch.randn(1, 7, 64, generator=g) * 2 + 0.5
    temb = torch.randn(1, 64, generator=g) * 0.3
    return ew, hidden, temb


def _final_reference(ew, hidden, temb):
    shift = ew["scale_shift_table"][:, 0] + temb
    scale = ew["scale_shift_table"][:, 1] + temb
    return torch.nn.functional.layer_norm(hidden, (64,), eps=1e-6) * (1 + scale[:, None]) \
        + shift[:, None]


def test_final_layer_is_layer_norm_scale_then_shift_from_the_table():
    """norm_out (:1031-1044): (shift, scale) = scale_shift_table + temb in that order, a
    LayerNorm without affine; proj_out identity here."""
    ew, hidden, temb = _final_case()
    assert torch.allclose(owan.final_layer(ew, hidden, temb), _final_reference(ew, hidden, temb),
                          atol=1e-5, rtol=1e-5)


def test_planted_swapped_shift_and_scale_in_the_final_layer_is_seen():
    ew, hidden, temb = _final_case()
    ref = _final_reference(ew, hidden, temb)
    swapped = dict(ew, scale_shift_table=ew["scale_shift_table"].flip(1))
    assert not torch.allclose(owan.final_layer(swapped, hidden, temb), ref, atol=1e-3)


def test_step_without_blocks_is_patch_embed_final_layer_unpatchify():
    """forward() with no blocks: the patch Conv3d, the conditioning's temb, the final layer and
    the unpatchify reshape, composed in that order (:932-1068)."""
    from difflet_amd.dit.wan import unpatchify

    ew, _, _ = _final_case(5)
    g = torch.Generator().manual_seed(6)
    lat = torch.randn(1, 16, 2, 4, 6, generator=g)
    t = torch.tensor([421.5])
    text = torch.randn(1, 3, 64, generator=g)
    out = owan.forward(FINAL, 0, lat, t, text, weights=(ew, []))
    tokens = torch.nn.functional.conv3d(lat, ew["patch_embedding.weight"],
                                        ew["patch_embedding.bias"], stride=(1, 2, 2))
    tokens = tokens.flatten(2).transpose(1, 2)
    temb, _, _ = owan.condition(ew, t, text)
    ref = unpatchify(_final_reference(ew, tokens, temb)[0], (2, 2, 3), (1, 2, 2))
    assert out.shape == lat.shape
    assert torch.allclose(out, ref, atol=1e-5, rtol=1e-5)
