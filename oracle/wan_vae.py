"""Wan's 3D causal VAE decoder restated in fp32 on the CPU, with seeded random weights. Test
infrastructure only (see oracle/__init__.py).

The reference decodes with ``WanVAEDecoderModel`` (difflet/models/wan/vae/modeling_vae.py:509-560),
its restatement of diffusers' ``AutoencoderKLWan`` decoder (diffusers 0.38.0, pinned in the
reference's pyproject.toml; absent here), which the CUDA flow calls as ``vae.decode`` in the
model dtype (difflet/backends/cuda/wan/application.py:115-134) after the pipeline's
``latents * std + mean`` (difflet/models/wan/pipeline.py:544-554). Qwen-Image decodes its one
latent frame with the same decoder (difflet/models/wan/vae/regions.py:3-6). The algorithm:

  post_quant_conv 1x1x1 over the whole latent video, then the decoder one latent frame at a
  time (a "chunk"), each causal 3x3x3 convolution reading a two-frame cache of its own input
  from the chunks before (modeling_vae.py:95-135, 225-268), then the clamp to [-1, 1]
  decoder: conv_in (z -> 4 base), mid block (resnet, attention, resnet), up blocks over
          dims = base * [m[-1]] + reversed(m), each num_res_blocks + 1 resnets then a resampler
          (upsample3d where the temporal flag is set, upsample2d otherwise, none after the last),
          the input channel count of blocks after the first halved by the resampler before
          (:436-470); RMS norm + SiLU, conv_out
  resnet: shortcut (1x1x1 conv when the width changes), RMS norm + SiLU, causal conv1, RMS norm +
          SiLU, causal conv2, plus the shortcut (:225-268)
  RMS norm (WanRMSNorm, :137-160): F.normalize over channels (x / max(||x||, 1e-12)) times
          sqrt(C) times gamma
  attention (WanAttentionBlock, :300-330): per frame, RMS norm, to_qkv 1x1, one head over the
          frame's pixels with all C channels (SDPA, scale 1/sqrt(C)), proj 1x1, residual
  upsample3d (WanResample, :163-222): the time convolution (3,1,1) C -> 2C, skipped on the first
          chunk ("Rep"), whose output frames interleave as (frame t, channels [0:C]) then (frame
          t, channels [C:2C]); then per frame nearest 2x and a 3x3 Conv2d C -> C/2
  upsample2d: per frame nearest 2x and a 3x3 Conv2d C -> C/2

`decode` follows the chunked algorithm step by step; `decode_sequence` states the same decoder
over the whole frame sequence at once (every causal convolution zero-pads two frames in front
of its level's frame sequence; the time convolution runs over frames 1.. with two zero frames
before frame 1 and frame 0 passes through). They are two derivations of one function: each pins
the other (tests/test_oracle_wan_vae.py).

`store` (a dtype or None) rounds the activations where a device that keeps them in that dtype
stores them (ops.rounder). Weights: N(0, fan_in^-1/2) convolutions, N(0, 0.02) biases, RMS norm
gammas 1 + N(0, 0.1), one generator per parameter.
"""

from __future__ import annotations

import dataclasses
import math

import torch
import torch.nn.functional as F

from oracle import ops

CACHE_T = 2  # frames of a causal convolution's input kept for the next chunk (modeling_vae.py:29)
REP = "Rep"  # a time convolution that has seen one chunk, so far skipped (modeling_vae.py:202-204)


@dataclasses.dataclass(frozen=True)
class WanVaeShape:
    """WanVAEDecoderConfig's fields that shape the decoder (modeling_vae.py:43-76)."""

    base_dim: int = 96
    z_dim: int = 16
    dim_mult: tuple = (1, 2, 4, 4)
    num_res_blocks: int = 2
    temperal_downsample: tuple = (False, True, True)
    out_channels: int = 3
    eps: float = 1e-12  # F.normalize's

    @property
    def temperal_upsample(self) -> tuple:
        return tuple(reversed(self.temperal_downsample))

    @property
    def dims(self) -> list[int]:
        """dims = base * [dim_mult[-1]] + base * reversed(dim_mult) (modeling_vae.py:436)."""
        m = list(self.dim_mult)
        return [self.base_dim * u for u in [m[-1]] + m[::-1]]


WAN_VAE = WanVaeShape()


def plan(shape: WanVaeShape) -> list[tuple[int, int, int, str | None]]:
    """Up blocks in order: (index, in channels, out channels, resample mode or None)
    (modeling_vae.py:437-456)."""
    dims, out = shape.dims, []
    n = len(shape.dim_mult)
    for i, (cin, cout) in enumerate(zip(dims[:-1], dims[1:])):
        if i > 0:
            cin = cin // 2
        up = i != n - 1
        mode = ("upsample3d" if shape.temperal_upsample[i] else "upsample2d") if up else None
        out.append((i, cin, cout, mode))
    return out


def param_shapes(shape: WanVaeShape) -> list[tuple[str, tuple]]:
    """AutoencoderKLWan's decoder keys and post_quant_conv (the reference's state dict, key for
    key: tests/unit/models/wan/test_modeling_wan_vae.py:97-121)."""
    z, top = shape.z_dim, shape.dims[0]
    p = [("post_quant_conv.weight", (z, z, 1, 1, 1)), ("post_quant_conv.bias", (z,)),
         ("decoder.conv_in.weight", (top, z, 3, 3, 3)), ("decoder.conv_in.bias", (top,))]

    def resnet(pre, cin, cout):
        q = [(f"{pre}.norm1.gamma", (cin, 1, 1, 1)),
             (f"{pre}.conv1.weight", (cout, cin, 3, 3, 3)), (f"{pre}.conv1.bias", (cout,)),
             (f"{pre}.norm2.gamma", (cout, 1, 1, 1)),
             (f"{pre}.conv2.weight", (cout, cout, 3, 3, 3)), (f"{pre}.conv2.bias", (cout,))]
        if cin != cout:
            q += [(f"{pre}.conv_shortcut.weight", (cout, cin, 1, 1, 1)),
                  (f"{pre}.conv_shortcut.bias", (cout,))]
        return q

    p += resnet("decoder.mid_block.resnets.0", top, top)
    a = "decoder.mid_block.attentions.0"
    p += [(f"{a}.norm.gamma", (top, 1, 1)), (f"{a}.to_qkv.weight", (3 * top, top, 1, 1)),
          (f"{a}.to_qkv.bias", (3 * top,)), (f"{a}.proj.weight", (top, top, 1, 1)),
          (f"{a}.proj.bias", (top,))]
    p += resnet("decoder.mid_block.resnets.1", top, top)
    for i, cin, cout, mode in plan(shape):
        c = cin
        for j in range(shape.num_res_blocks + 1):
            p += resnet(f"decoder.up_blocks.{i}.resnets.{j}", c, cout)
            c = cout
        if mode is not None:
            u = f"decoder.up_blocks.{i}.upsamplers.0"
            p += [(f"{u}.resample.1.weight", (cout // 2, cout, 3, 3)),
                  (f"{u}.resample.1.bias", (cout // 2,))]
            if mode == "upsample3d":
                p += [(f"{u}.time_conv.weight", (2 * cout, cout, 3, 1, 1)),
                      (f"{u}.time_conv.bias", (2 * cout,))]
    last = shape.dims[-1]
    p += [("decoder.norm_out.gamma", (last, 1, 1, 1)),
          ("decoder.conv_out.weight", (shape.out_channels, last, 3, 3, 3)),
          ("decoder.conv_out.bias", (shape.out_channels,))]
    return p


def weights(shape: WanVaeShape, seed: int, dtype: torch.dtype | None = None) -> dict[str, torch.Tensor]:
    """fp32 parameters, rounded through `dtype` when given (a model loaded in that dtype)."""
    r = ops.rounder(dtype)
    out = {}
    for idx, (name, shp) in enumerate(param_shapes(shape)):
        g = torch.Generator().manual_seed(seed * 7919 + idx)
        x = torch.randn(shp, generator=g, dtype=torch.float32)
        if name.endswith("gamma"):
            x = 1.0 + 0.1 * x
        elif name.endswith("bias"):
            x = 0.02 * x
        else:
            x = x * (math.prod(shp[1:]) ** -0.5)
        out[name] = r(x)
    return out


def rms_norm(x, gamma, shape: WanVaeShape):
    """WanRMSNorm (modeling_vae.py:154-160) over dim 1 in fp32: F.normalize, times sqrt(C) and
    gamma (the bias is 0.0: bias=False throughout the decoder)."""
    c = x.shape[1]
    return F.normalize(x.float(), dim=1, eps=shape.eps) * math.sqrt(c) * gamma


def _norm_silu(w, name, x, shape, r):
    """RMS norm then SiLU, stored once (the device computes both in fp32 and rounds the result;
    storing the norm's output as well moves the bf16 decode by 1.8e-2 on the small decoder)."""
    return r(F.silu(rms_norm(x, w[name], shape)))


def causal_conv(x, wt, b, cache=None):
    """WanCausalConv3d.forward (modeling_vae.py:121-134) for kernel 3 or 1: the cache frames (if
    any) prepended, zeros for the rest of the 2 * padding frames in front, spatial zero padding."""
    kt = wt.shape[2]
    pt, ps = kt - 1, wt.shape[3] // 2
    if cache is not None and pt > 0:
        x = torch.cat([cache, x], dim=2)
        pt -= cache.shape[2]
    return F.conv3d(F.pad(x, (ps, ps, ps, ps, pt, 0)), wt, b)


def _tail(x, old):
    """The next cache of a causal convolution that read `x` after the cache `old`
    (modeling_vae.py:31-33, 244-250): the last two frames of x, with the last frame of `old`
    prepended when x has one frame and `old` exists."""
    t = x[:, :, -CACHE_T:].clone()
    if t.shape[2] < CACHE_T and old is not None:
        t = torch.cat([old[:, :, -1:], t], dim=2)
    return t


class _Walk:
    """One chunk's pass through the decoder: the convolution caches live in `cache` (keyed by the
    convolution's name) across chunks, as feat_cache does by position."""

    def __init__(self, w, shape: WanVaeShape, cache: dict, r):
        self.w, self.shape, self.cache, self.r = w, shape, cache, r

    def conv(self, name, x):
        old = self.cache.get(name)
        y = causal_conv(x, self.w[f"{name}.weight"], self.w[f"{name}.bias"], old)
        self.cache[name] = _tail(x, old)
        return self.r(y)

    def resnet(self, pre, x):
        w, r = self.w, self.r
        h = x
        if f"{pre}.conv_shortcut.weight" in w:
            h = r(causal_conv(x, w[f"{pre}.conv_shortcut.weight"], w[f"{pre}.conv_shortcut.bias"]))
        y = _norm_silu(w, f"{pre}.norm1.gamma", x, self.shape, r)
        y = self.conv(f"{pre}.conv1", y)
        y = _norm_silu(w, f"{pre}.norm2.gamma", y, self.shape, r)
        old = self.cache.get(f"{pre}.conv2")
        y2 = causal_conv(y, w[f"{pre}.conv2.weight"], w[f"{pre}.conv2.bias"], old)
        self.cache[f"{pre}.conv2"] = _tail(y, old)
        return r(y2 + h)

    def attention(self, pre, x):
        return attention(self.w, pre, x, self.shape, self.r)

    def resample(self, pre, mode, x):
        w, r = self.w, self.r
        b, c, t, hh, ww = x.shape
        if mode == "upsample3d":
            name = f"{pre}.time_conv"
            st = self.cache.get(name)
            if st is None:
                self.cache[name] = REP
            else:
                tail = x[:, :, -CACHE_T:].clone()
                if tail.shape[2] < CACHE_T:
                    head = torch.zeros_like(tail) if st is REP else st[:, :, -1:]
                    tail = torch.cat([head, tail], dim=2)
                y = causal_conv(x, w[f"{name}.weight"], w[f"{name}.bias"],
                                None if st is REP else st)
                self.cache[name] = tail
                x = interleave_time(r(y))
        return spatial_upsample(w, pre, x, r)


def interleave_time(y):
    """The time convolution's [B, 2C, T, H, W] output as [B, C, 2T, H, W]: frame 2t takes
    channels [0:C] of frame t, frame 2t + 1 channels [C:2C] (modeling_vae.py:219-221)."""
    b, c2, t, hh, ww = y.shape
    c = c2 // 2
    y = y.reshape(b, 2, c, t, hh, ww)
    return torch.stack((y[:, 0], y[:, 1]), dim=3).reshape(b, c, 2 * t, hh, ww)


def spatial_upsample(w, pre, x, r):
    """Per frame: nearest 2x, then the 3x3 Conv2d (WanResample.resample, modeling_vae.py:223-226)."""
    b, c, t, hh, ww = x.shape
    f = x.permute(0, 2, 1, 3, 4).reshape(b * t, c, hh, ww)
    f = F.interpolate(f, scale_factor=2.0, mode="nearest")
    f = r(F.conv2d(f, w[f"{pre}.resample.1.weight"], w[f"{pre}.resample.1.bias"], padding=1))
    return f.reshape(b, t, f.shape[1], 2 * hh, 2 * ww).permute(0, 2, 1, 3, 4)


def attention(w, pre, x, shape: WanVaeShape, r):
    """WanAttentionBlock.forward (modeling_vae.py:312-330): per frame, one head over the
    frame's pixels with every channel, SDPA's default scale 1/sqrt(C)."""
    b, c, t, hh, ww = x.shape
    f = x.permute(0, 2, 1, 3, 4).reshape(b * t, c, hh, ww)
    n = r(rms_norm(f, w[f"{pre}.norm.gamma"], shape))
    qkv = r(F.conv2d(n, w[f"{pre}.to_qkv.weight"], w[f"{pre}.to_qkv.bias"]))
    qkv = qkv.reshape(b * t, 3 * c, hh * ww).transpose(1, 2)  # [frames, pixels, 3C]
    q, k, v = qkv[..., :c], qkv[..., c:2 * c], qkv[..., 2 * c:]
    p = r(torch.softmax((q @ k.transpose(1, 2)) / math.sqrt(c), dim=-1))
    o = r(p @ v).transpose(1, 2).reshape(b * t, c, hh, ww)
    o = F.conv2d(o, w[f"{pre}.proj.weight"], w[f"{pre}.proj.bias"])
    o = o.reshape(b, t, c, hh, ww).permute(0, 2, 1, 3, 4)
    return r(o + x)


def _decoder_chunk(walk: _Walk, x):
    """WanDecoder3d.forward (modeling_vae.py:473-506) on one chunk."""
    shape = walk.shape
    x = walk.conv("decoder.conv_in", x)
    x = walk.resnet("decoder.mid_block.resnets.0", x)
    x = walk.attention("decoder.mid_block.attentions.0", x)
    x = walk.resnet("decoder.mid_block.resnets.1", x)
    for i, _, _, mode in plan(shape):
        for j in range(shape.num_res_blocks + 1):
            x = walk.resnet(f"decoder.up_blocks.{i}.resnets.{j}", x)
        if mode is not None:
            x = walk.resample(f"decoder.up_blocks.{i}.upsamplers.0", mode, x)
    x = _norm_silu(walk.w, "decoder.norm_out.gamma", x, shape, walk.r)
    return walk.conv("decoder.conv_out", x)


def post_quant(w, z, r):
    return r(causal_conv(r(z.float()), w["post_quant_conv.weight"], w["post_quant_conv.bias"]))


def decode(w: dict[str, torch.Tensor], shape: WanVaeShape, z: torch.Tensor, store=None) -> torch.Tensor:
    """Video [B, out_channels, 1 + 4 (T - 1), 8 h, 8 w] (two temporal upsamplings) from latents
    z [B, z_dim, T, h, w], chunk by chunk (WanVAEDecoderModel.forward, modeling_vae.py:545-557)."""
    r = ops.rounder(store)
    x = post_quant(w, z, r)
    cache: dict = {}
    walk = _Walk(w, shape, cache, r)
    frames = [_decoder_chunk(walk, x[:, :, i:i + 1]) for i in range(x.shape[2])]
    return torch.clamp(torch.cat(frames, dim=2), -1.0, 1.0)


# ---------------------------------------------------------------- whole-sequence form
def _seq_conv(w, name, x):
    return causal_conv(x, w[f"{name}.weight"], w[f"{name}.bias"])


def _seq_resnet(w, pre, x, shape, r):
    h = x
    if f"{pre}.conv_shortcut.weight" in w:
        h = r(_seq_conv(w, f"{pre}.conv_shortcut", x))
    y = _norm_silu(w, f"{pre}.norm1.gamma", x, shape, r)
    y = r(_seq_conv(w, f"{pre}.conv1", y))
    y = _norm_silu(w, f"{pre}.norm2.gamma", y, shape, r)
    return r(_seq_conv(w, f"{pre}.conv2", y) + h)


def decode_sequence(w: dict[str, torch.Tensor], shape: WanVaeShape, z: torch.Tensor,
                    store=None) -> torch.Tensor:
    """The same decode over whole frame sequences: each causal convolution pads its level's
    sequence with two zero frames in front; a time convolution maps frames 1.. (two zero frames
    before frame 1) and frame 0 passes through unchanged."""
    r = ops.rounder(store)
    x = post_quant(w, z, r)
    x = r(_seq_conv(w, "decoder.conv_in", x))
    x = _seq_resnet(w, "decoder.mid_block.resnets.0", x, shape, r)
    x = attention(w, "decoder.mid_block.attentions.0", x, shape, r)
    x = _seq_resnet(w, "decoder.mid_block.resnets.1", x, shape, r)
    for i, _, _, mode in plan(shape):
        for j in range(shape.num_res_blocks + 1):
            x = _seq_resnet(w, f"decoder.up_blocks.{i}.resnets.{j}", x, shape, r)
        if mode is None:
            continue
        pre = f"decoder.up_blocks.{i}.upsamplers.0"
        if mode == "upsample3d" and x.shape[2] > 1:
            rest = interleave_time(r(_seq_conv(w, f"{pre}.time_conv", x[:, :, 1:])))
            x = torch.cat([x[:, :, :1], rest], dim=2)
        x = spatial_upsample(w, pre, x, r)
    x = _norm_silu(w, "decoder.norm_out.gamma", x, shape, r)
    x = r(_seq_conv(w, "decoder.conv_out", x))
    return torch.clamp(x, -1.0, 1.0)


def denormalize(latents: torch.Tensor, mean, std) -> torch.Tensor:
    """latents * std + mean per channel when the config has both (pipeline.py:544-554)."""
    if mean is None or std is None or len(mean) == 0 or len(std) == 0:
        return latents
    m = torch.tensor(mean, dtype=latents.dtype).view(1, -1, 1, 1, 1)
    s = torch.tensor(std, dtype=latents.dtype).view(1, -1, 1, 1, 1)
    return latents * s + m
