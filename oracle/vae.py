"""FLUX's VAE decoder restated in fp32 on the CPU, with seeded random weights. Test
infrastructure only (see oracle/__init__.py).

The reference decodes with diffusers' 2D ``Decoder`` (diffusers 0.38.0, pinned in its
pyproject.toml; absent here), built from the VAE config by get_decoder_config
(difflet/models/flux/vae/modeling_vae.py:107-117) with GroupNorm in fp32 (PatchedGroupNorm,
:39-68) and no post_quant_conv for FLUX.1 (difflet/backends/neuron/flux/vae.py:25-36), fed
latents / scaling_factor + shift_factor (difflet/models/flux/pipeline.py:448-449). The decoder's
published algorithm, restated here with torch's own convolution, GroupNorm and nearest
interpolation:
  conv_in 3x3 (latent -> top channels)
  mid block: resnet, attention (GroupNorm, one head over all channels, q/k/v/out linears with
             bias, softmax scale 1/sqrt(channels), residual), resnet
  up blocks over the reversed channel list, each layers_per_block + 1 resnets (the first may
             change the channel count, with a 1x1 shortcut), then (all but the last) nearest 2x
             upsampling followed by a 3x3 conv
  GroupNorm + SiLU, conv_out 3x3
  resnet: GroupNorm + SiLU, conv1 3x3, GroupNorm + SiLU, conv2 3x3, plus the input (or its 1x1
          shortcut); GroupNorm eps 1e-6 and 32 groups throughout.

`store` (a dtype or None) rounds the activations where a device that keeps them in that dtype
stores them (ops.rounder). Weights: N(0, fan_in^-1/2) convolutions and linears, N(0, 0.02)
biases, GroupNorm weights 1 + N(0, 0.1) and biases N(0, 0.1), one generator per parameter.
"""

from __future__ import annotations

import dataclasses
import math

import torch
import torch.nn.functional as F

from oracle import ops


@dataclasses.dataclass(frozen=True)
class VaeShape:
    latent_channels: int = 16
    out_channels: int = 3
    block_out_channels: tuple = (128, 256, 512, 512)
    layers_per_block: int = 2
    groups: int = 32
    eps: float = 1e-6
    scaling_factor: float = 0.3611
    shift_factor: float = 0.1159


FLUX_VAE = VaeShape()


def plan(shape: VaeShape) -> list[tuple[int, int, int, bool]]:
    """(up block, resnet, in channels, out channels) and whether the block upsamples, in order:
    [(i, j, cin, cout, upsample_after)] with upsample_after set on each block's last resnet."""
    rev = list(reversed(shape.block_out_channels))
    out, prev = [], rev[0]
    for i, c in enumerate(rev):
        for j in range(shape.layers_per_block + 1):
            cin = prev if j == 0 else c
            out.append((i, j, cin, c, j == shape.layers_per_block and i < len(rev) - 1))
        prev = c
    return out


def param_shapes(shape: VaeShape) -> list[tuple[str, tuple]]:
    """diffusers AutoencoderKL decoder keys (the reference loads them key for key)."""
    top = shape.block_out_channels[-1]
    p = [("decoder.conv_in.weight", (top, shape.latent_channels, 3, 3)),
         ("decoder.conv_in.bias", (top,))]

    def resnet(pre, cin, cout):
        q = [(f"{pre}.norm1.weight", (cin,)), (f"{pre}.norm1.bias", (cin,)),
             (f"{pre}.conv1.weight", (cout, cin, 3, 3)), (f"{pre}.conv1.bias", (cout,)),
             (f"{pre}.norm2.weight", (cout,)), (f"{pre}.norm2.bias", (cout,)),
             (f"{pre}.conv2.weight", (cout, cout, 3, 3)), (f"{pre}.conv2.bias", (cout,))]
        if cin != cout:
            q += [(f"{pre}.conv_shortcut.weight", (cout, cin, 1, 1)), (f"{pre}.conv_shortcut.bias", (cout,))]
        return q

    p += resnet("decoder.mid_block.resnets.0", top, top)
    a = "decoder.mid_block.attentions.0"
    p += [(f"{a}.group_norm.weight", (top,)), (f"{a}.group_norm.bias", (top,))]
    for n in ("to_q", "to_k", "to_v", "to_out.0"):
        p += [(f"{a}.{n}.weight", (top, top)), (f"{a}.{n}.bias", (top,))]
    p += resnet("decoder.mid_block.resnets.1", top, top)
    for i, j, cin, cout, up in plan(shape):
        p += resnet(f"decoder.up_blocks.{i}.resnets.{j}", cin, cout)
        if up:
            p += [(f"decoder.up_blocks.{i}.upsamplers.0.conv.weight", (cout, cout, 3, 3)),
                  (f"decoder.up_blocks.{i}.upsamplers.0.conv.bias", (cout,))]
    c0 = shape.block_out_channels[0]
    p += [("decoder.conv_norm_out.weight", (c0,)), ("decoder.conv_norm_out.bias", (c0,)),
          ("decoder.conv_out.weight", (shape.out_channels, c0, 3, 3)),
          ("decoder.conv_out.bias", (shape.out_channels,))]
    return p


def weights(shape: VaeShape, seed: int, dtype: torch.dtype | None = None) -> dict[str, torch.Tensor]:
    """fp32 parameters; the conv / linear weights and biases rounded through `dtype` when given
    (GroupNorm affine vectors stay fp32, as PatchedGroupNorm keeps them)."""
    r = ops.rounder(dtype)
    out = {}
    for idx, (name, shp) in enumerate(param_shapes(shape)):
        g = torch.Generator().manual_seed(seed * 7919 + idx)
        x = torch.randn(shp, generator=g, dtype=torch.float32)
        if "norm" in name:
            out[name] = 1.0 + 0.1 * x if name.endswith("weight") else 0.1 * x
            continue
        if name.endswith("bias"):
            x = 0.02 * x
        else:
            x = x * (math.prod(shp[1:]) ** -0.5)
        out[name] = r(x)
    return out


def group_norm(x, w, b, shape: VaeShape):
    """PatchedGroupNorm (modeling_vae.py:66-68): F.group_norm in fp32."""
    return F.group_norm(x.float(), shape.groups, w, b, shape.eps)


def conv(x, w, b, pad=1):
    return F.conv2d(x, w, b, padding=pad)


def resnet(w, pre, x, shape: VaeShape, r):
    h = r(F.silu(group_norm(x, w[f"{pre}.norm1.weight"], w[f"{pre}.norm1.bias"], shape)))
    h = r(conv(h, w[f"{pre}.conv1.weight"], w[f"{pre}.conv1.bias"]))
    h = r(F.silu(group_norm(h, w[f"{pre}.norm2.weight"], w[f"{pre}.norm2.bias"], shape)))
    sc = x
    if f"{pre}.conv_shortcut.weight" in w:
        sc = r(conv(x, w[f"{pre}.conv_shortcut.weight"], w[f"{pre}.conv_shortcut.bias"], pad=0))
    return r(sc + conv(h, w[f"{pre}.conv2.weight"], w[f"{pre}.conv2.bias"]))


def attention(w, pre, x, shape: VaeShape, r):
    """The mid block's Attention (one head of all channels, group_norm first, residual)."""
    b, c, hh, ww = x.shape
    n = r(group_norm(x, w[f"{pre}.group_norm.weight"], w[f"{pre}.group_norm.bias"], shape))
    t = n.reshape(b, c, hh * ww).transpose(1, 2)
    lin = lambda z, nm: z @ w[f"{pre}.{nm}.weight"].T + w[f"{pre}.{nm}.bias"]  # noqa: E731
    q, k, v = r(lin(t, "to_q")), r(lin(t, "to_k")), r(lin(t, "to_v"))
    p = r(torch.softmax((q @ k.transpose(1, 2)) / math.sqrt(c), dim=-1))
    o = r(p @ v)
    out = lin(o, "to_out.0").transpose(1, 2).reshape(b, c, hh, ww)
    return r(out + x)


def decode(w: dict[str, torch.Tensor], shape: VaeShape, z: torch.Tensor, store=None) -> torch.Tensor:
    """Images [B, out_channels, 8 h, 8 w] from unscaled latents z [B, latent_channels, h, w]."""
    r = ops.rounder(store)
    x = r(conv(r(z.float()), w["decoder.conv_in.weight"], w["decoder.conv_in.bias"]))
    x = resnet(w, "decoder.mid_block.resnets.0", x, shape, r)
    x = attention(w, "decoder.mid_block.attentions.0", x, shape, r)
    x = resnet(w, "decoder.mid_block.resnets.1", x, shape, r)
    for i, j, _, _, up in plan(shape):
        x = resnet(w, f"decoder.up_blocks.{i}.resnets.{j}", x, shape, r)
        if up:
            x = F.interpolate(x, scale_factor=2.0, mode="nearest")
            x = r(conv(x, w[f"decoder.up_blocks.{i}.upsamplers.0.conv.weight"],
                       w[f"decoder.up_blocks.{i}.upsamplers.0.conv.bias"]))
    x = r(F.silu(group_norm(x, w["decoder.conv_norm_out.weight"], w["decoder.conv_norm_out.bias"], shape)))
    return r(conv(x, w["decoder.conv_out.weight"], w["decoder.conv_out.bias"]))


def unscale(latents: torch.Tensor, shape: VaeShape) -> torch.Tensor:
    """pipeline.py:448: latents / scaling_factor + shift_factor."""
    return latents / shape.scaling_factor + shape.shift_factor
