"""Pins of the VAE decoder oracle (oracle/vae.py) and the decoder's host logic, on the CPU.

diffusers (0.38.0, the reference's pin) is absent, so the decoder's composition is restated from
its published algorithm. What pins it: torch's own GroupNorm module, nearest interpolation and
scaled-dot-product attention for the pieces (the reference's own test holds PatchedGroupNorm
equal to nn.GroupNorm: tests/unit/models/flux/test_flux_vae.py:43-47); the scale factor of
modeling_vae.py:120-127; and a closed-form reduction of the whole decoder (every resnet's
second conv and the attention's output projection zeroed, so each block passes its input, or
its 1x1 shortcut, through) against a chain of torch operations. Each pin is paired with a
planted mistake in the oracle that it catches. The im2col column order and weight packing of
the device path are checked against F.conv2d.
"""

import dataclasses
import math

import pytest
import torch
import torch.nn.functional as F

from difflet_amd.vae import decoder as dvae
from oracle import vae as ovae

SMALL = ovae.VaeShape(latent_channels=4, block_out_channels=(32, 32, 64, 64), layers_per_block=1)


def rel_l2(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def _z(shape, h=6, w=5, seed=1):
    return torch.randn(1, shape.latent_channels, h, w, generator=torch.Generator().manual_seed(seed))


def test_layout_scale_factor_and_plan():
    assert dict(ovae.param_shapes(ovae.FLUX_VAE)) == dvae.param_shapes(dvae.FLUX_VAE)
    assert dvae.FLUX_VAE.scale_factor == 8  # 2 ** (len(block_out_channels) - 1)
    plan = ovae.plan(ovae.FLUX_VAE)
    assert [(i, j, cin, cout) for i, j, cin, cout, _ in plan if cin != cout] == [(2, 0, 512, 256),
                                                                               (3, 0, 256, 128)]
    assert [i for i, _, _, _, up in plan if up] == [0, 1, 2]
    out = ovae.decode(ovae.weights(SMALL, 1), SMALL, _z(SMALL))
    assert out.shape == (1, 3, 6 * 8, 5 * 8)


def test_group_norm_is_torch_group_norm():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 64, 7, 9, generator=g) * 3 + 1
    mod = torch.nn.GroupNorm(32, 64, eps=1e-6)
    with torch.no_grad():
        mod.weight.copy_(torch.randn(64, generator=g))
        mod.bias.copy_(torch.randn(64, generator=g))
    ref = mod(x)
    assert torch.allclose(ovae.group_norm(x, mod.weight, mod.bias, SMALL), ref, atol=1e-5)


def test_attention_block_is_sdpa_with_residual(monkeypatch):
    """x + to_out(SDPA(q, k, v)) over GroupNorm(x), one head of all channels."""
    shape = SMALL
    w = ovae.weights(shape, 3)
    pre = "decoder.mid_block.attentions.0"
    x = torch.randn(1, 64, 6, 5, generator=torch.Generator().manual_seed(3))
    gn = torch.nn.GroupNorm(32, 64, eps=1e-6)
    with torch.no_grad():
        gn.weight.copy_(w[f"{pre}.group_norm.weight"])
        gn.bias.copy_(w[f"{pre}.group_norm.bias"])
    t = gn(x).reshape(1, 64, 30).transpose(1, 2)
    lin = lambda z, n: F.linear(z, w[f"{pre}.{n}.weight"], w[f"{pre}.{n}.bias"])  # noqa: E731
    o = F.scaled_dot_product_attention(lin(t, "to_q")[:, None], lin(t, "to_k")[:, None],
                                       lin(t, "to_v")[:, None])[:, 0]
    ref = lin(o, "to_out.0").transpose(1, 2).reshape(1, 64, 6, 5) + x
    ident = lambda v: v  # noqa: E731
    got = ovae.attention(w, pre, x, shape, ident)
    assert rel_l2(got, ref) < 1e-6
    # planted: softmax scale 1 / C instead of 1 / sqrt(C)
    monkeypatch.setattr(ovae.math, "sqrt", lambda c: c)
    assert rel_l2(ovae.attention(w, pre, x, shape, ident), ref) > 1e-3


def _passthrough_weights(shape, seed):
    """Every resnet's conv2 and the attention's output projection zeroed: each resnet returns
    its input (or its 1x1 shortcut), the attention its input."""
    w = ovae.weights(shape, seed)
    for k in w:
        if ".conv2." in k or ".to_out.0." in k:
            w[k] = torch.zeros_like(w[k])
    return w


def _passthrough_chain(w, shape, z):
    """The reduced decoder by torch operations alone: conv_in, then per up block its first
    resnet's shortcut (where the channels change) and (all but the last) nearest 2x + conv,
    then GroupNorm + SiLU + conv_out."""
    x = F.conv2d(z, w["decoder.conv_in.weight"], w["decoder.conv_in.bias"], padding=1)
    for i in range(len(shape.block_out_channels)):
        sc = f"decoder.up_blocks.{i}.resnets.0.conv_shortcut"
        if f"{sc}.weight" in w:
            x = F.conv2d(x, w[f"{sc}.weight"], w[f"{sc}.bias"])
        if i < len(shape.block_out_channels) - 1:
            x = F.interpolate(x, scale_factor=2.0, mode="nearest")
            up = f"decoder.up_blocks.{i}.upsamplers.0.conv"
            x = F.conv2d(x, w[f"{up}.weight"], w[f"{up}.bias"], padding=1)
    gn = torch.nn.GroupNorm(shape.groups, x.shape[1], eps=shape.eps)
    with torch.no_grad():
        gn.weight.copy_(w["decoder.conv_norm_out.weight"])
        gn.bias.copy_(w["decoder.conv_norm_out.bias"])
    x = torch.nn.SiLU()(gn(x))
    return F.conv2d(x, w["decoder.conv_out.weight"], w["decoder.conv_out.bias"], padding=1)


def test_decoder_reduces_to_the_passthrough_chain():
    w = _passthrough_weights(SMALL, 4)
    z = _z(SMALL, seed=4)
    ref = _passthrough_chain(w, SMALL, z)
    assert rel_l2(ovae.decode(w, SMALL, z), ref) < 1e-5


def test_planted_bilinear_upsampling_is_caught(monkeypatch):
    w = _passthrough_weights(SMALL, 4)
    z = _z(SMALL, seed=4)
    ref = _passthrough_chain(w, SMALL, z)
    real = F.interpolate
    monkeypatch.setattr(ovae.F, "interpolate",
                        lambda x, scale_factor, mode: real(x, scale_factor=scale_factor,
                                                           mode="bilinear", align_corners=False))
    assert rel_l2(ovae.decode(w, SMALL, z), ref) > 1e-2


def test_planted_dropped_residual_is_caught(monkeypatch):
    w = _passthrough_weights(SMALL, 4)
    z = _z(SMALL, seed=4)
    ref = _passthrough_chain(w, SMALL, z)
    real = ovae.resnet

    def no_residual(w_, pre, x, shape, r):
        y = real(w_, pre, x, shape, r)
        sc = x
        if f"{pre}.conv_shortcut.weight" in w_:
            sc = F.conv2d(x, w_[f"{pre}.conv_shortcut.weight"], w_[f"{pre}.conv_shortcut.bias"])
        return y - sc

    monkeypatch.setattr(ovae, "resnet", no_residual)
    assert rel_l2(ovae.decode(w, SMALL, z), ref) > 1e-2


def test_planted_missing_output_silu_is_caught(monkeypatch):
    w = _passthrough_weights(SMALL, 4)
    z = _z(SMALL, seed=4)
    ref = _passthrough_chain(w, SMALL, z)
    real_silu = F.silu
    calls = {"n": 0}

    def last_silu_off(x):  # the decoder's last SiLU is conv_norm_out's
        calls["n"] += 1
        return x if x.shape[1] == SMALL.block_out_channels[0] and calls["n"] > 6 * 2 + 3 else real_silu(x)

    monkeypatch.setattr(ovae.F, "silu", last_silu_off)
    assert rel_l2(ovae.decode(w, SMALL, z), ref) > 1e-2


@pytest.mark.parametrize("cin,cout,kq", [(16, 512, 64), (32, 64, 64), (64, 3, 4), (8, 8, 4)])
def test_packed_weights_times_im2col_rows_are_the_convolution(cin, cout, kq):
    """The device's operand layout: weight [Cout][ky][kx][Cin] against rows of the 9 taps'
    channels (tap 3 ky + kx, zero outside the image), with the padding of the GEMM multiples,
    equals F.conv2d(padding=1); with nearest 2x upsampling first, F.interpolate then conv."""
    g = torch.Generator().manual_seed(cin + cout)
    x = torch.randn(1, cin, 5, 7, generator=g)
    w = torch.randn(cout, cin, 3, 3, generator=g)
    b = torch.randn(cout, generator=g)
    wp, bp, co, kp = dvae.pack_conv(w, b, kq, torch.float32)
    assert co == cout and wp.shape == (-(-cout // 4) * 4, -(-9 * cin // kq) * kq) and kp == wp.shape[1]
    for up in (False, True):
        xi = F.interpolate(x, scale_factor=2.0, mode="nearest") if up else x
        h, wd = xi.shape[2:]
        hwc = F.pad(xi[0].permute(1, 2, 0), (0, 0, 1, 1, 1, 1))  # [h + 2, w + 2, C]
        rows = torch.stack([hwc[ky:ky + h, kx:kx + wd] for ky in range(3) for kx in range(3)], 2)
        cols = F.pad(rows.reshape(h * wd, 9 * cin), (0, kp - 9 * cin))
        y = (cols @ wp.T + bp)[:, :cout].reshape(h, wd, cout).permute(2, 0, 1)
        assert rel_l2(y, F.conv2d(xi, w, b, padding=1)[0]) < 1e-5


def test_vae_config_from_diffusers_dict():
    raw = {"latent_channels": 16, "out_channels": 3, "block_out_channels": [128, 256, 512, 512],
           "layers_per_block": 2, "norm_num_groups": 32, "act_fn": "silu",
           "up_block_types": ["UpDecoderBlock2D"] * 4, "mid_block_add_attention": True,
           "scaling_factor": 0.3611, "shift_factor": 0.1159, "use_post_quant_conv": False}
    assert dvae.VaeConfig.from_diffusers_dict(raw) == dvae.FLUX_VAE
    with pytest.raises(NotImplementedError):
        dvae.VaeConfig.from_diffusers_dict(dict(raw, act_fn="relu"))
    with pytest.raises(NotImplementedError):
        dvae.VaeDecoder(dataclasses.replace(dvae.FLUX_VAE, use_post_quant_conv=True),
                        lambda n: None, device="cpu")
    assert math.isclose(float(ovae.unscale(torch.tensor(0.3611), ovae.FLUX_VAE)), 1.1159, rel_tol=1e-6)
