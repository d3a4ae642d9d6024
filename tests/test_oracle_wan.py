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
