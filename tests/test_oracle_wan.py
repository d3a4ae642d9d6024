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
