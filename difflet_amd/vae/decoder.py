"""FLUX's VAE decoder on the gfx950 kernels: diffusers' 2D ``Decoder`` as the reference builds it
(get_decoder_config, difflet/models/flux/vae/modeling_vae.py:107-117; the application's
decode of unscaled latents, difflet/backends/neuron/flux/vae.py:25-36,78-80), bf16 or fp32 (the
reference runs fp32 by default, GroupNorm in fp32 either way: modeling_vae.py:39-68).

Activations stay channels-last, [pixels][channels] per image, so a 3x3 convolution is the GEMM
of its im2col rows (the nearest 2x upsampling of Upsample2D folded into their addressing) with
the weight repacked [Cout][ky][kx][Cin] once at load, bias and any residual added in the GEMM's
epilogue: one implicit GEMM that gathers the rows stage by stage (kernels.conv_causal on one
frame; bf16 on the bf16 matrix cores, fp32 on the fp32 GEMM). GroupNorm (+ SiLU) is its own two-pass kernel. The mid block's attention
(one head of 512 channels over the latent's pixels) runs as GEMMs: fp32 scores S = Q K^T, the
row softmax kernel, P V, then the output projection with the residual.

Per resnet: GroupNorm+SiLU -> conv1 -> GroupNorm+SiLU -> conv2 (+ bias + shortcut), the shortcut
a 1x1 GEMM where the channel count changes.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Callable

import torch

from difflet_amd import _lib, kernels


@dataclasses.dataclass(frozen=True)
class VaeConfig:
    """The decoder half of an AutoencoderKL config (diffusers names)."""

    latent_channels: int = 16
    out_channels: int = 3
    block_out_channels: tuple = (128, 256, 512, 512)
    layers_per_block: int = 2
    norm_num_groups: int = 32
    scaling_factor: float = 0.3611
    shift_factor: float = 0.1159
    use_post_quant_conv: bool = False

    @property
    def scale_factor(self) -> int:
        """2 ** (len(block_out_channels) - 1) (modeling_vae.py:120-127)."""
        return 2 ** (len(self.block_out_channels) - 1)

    @classmethod
    def from_diffusers_dict(cls, raw: dict) -> "VaeConfig":
        """From the VAE's config.json. The standard Decoder only, with SiLU, UpDecoderBlock2D
        blocks and the mid-block attention (FLUX.1's VAE)."""
        ups = raw.get("up_block_types", ["UpDecoderBlock2D"] * len(raw.get("block_out_channels", (0,) * 4)))
        if any(u != "UpDecoderBlock2D" for u in ups) or raw.get("act_fn", "silu") != "silu" \
                or not raw.get("mid_block_add_attention", True):
            raise NotImplementedError("only the standard Decoder (UpDecoderBlock2D, SiLU, mid-block "
                                      "attention) is supported")
        return cls(latent_channels=int(raw.get("latent_channels", 16)),
                   out_channels=int(raw.get("out_channels", 3)),
                   block_out_channels=tuple(raw.get("block_out_channels", (128, 256, 512, 512))),
                   layers_per_block=int(raw.get("layers_per_block", 2)),
                   norm_num_groups=int(raw.get("norm_num_groups", 32)),
                   scaling_factor=float(raw.get("scaling_factor", 0.3611)),
                   shift_factor=float(raw.get("shift_factor", 0.1159) or 0.0),
                   use_post_quant_conv=bool(raw.get("use_post_quant_conv", True)))


FLUX_VAE = VaeConfig()
EPS = 1e-6  # the decoder's GroupNorm eps (resnets, attention, conv_norm_out)


def _plan(cfg: VaeConfig):
    """(up block, resnet, cin, cout, upsample after) in execution order."""
    rev = list(reversed(cfg.block_out_channels))
    out, prev = [], rev[0]
    for i, c in enumerate(rev):
        for j in range(cfg.layers_per_block + 1):
            out.append((i, j, prev if j == 0 else c, c,
                        j == cfg.layers_per_block and i < len(rev) - 1))
        prev = c
    return out


def param_shapes(cfg: VaeConfig) -> dict[str, tuple]:
    """diffusers AutoencoderKL decoder keys (the reference's checkpoint layout, key for key)."""
    top = cfg.block_out_channels[-1]
    p = {"decoder.conv_in.weight": (top, cfg.latent_channels, 3, 3), "decoder.conv_in.bias": (top,)}
    if cfg.use_post_quant_conv:
        p["post_quant_conv.weight"] = (cfg.latent_channels, cfg.latent_channels, 1, 1)
        p["post_quant_conv.bias"] = (cfg.latent_channels,)

    def resnet(pre, cin, cout):
        p.update({f"{pre}.norm1.weight": (cin,), f"{pre}.norm1.bias": (cin,),
                  f"{pre}.conv1.weight": (cout, cin, 3, 3), f"{pre}.conv1.bias": (cout,),
                  f"{pre}.norm2.weight": (cout,), f"{pre}.norm2.bias": (cout,),
                  f"{pre}.conv2.weight": (cout, cout, 3, 3), f"{pre}.conv2.bias": (cout,)})
        if cin != cout:
            p[f"{pre}.conv_shortcut.weight"] = (cout, cin, 1, 1)
            p[f"{pre}.conv_shortcut.bias"] = (cout,)

    resnet("decoder.mid_block.resnets.0", top, top)
    a = "decoder.mid_block.attentions.0"
    p[f"{a}.group_norm.weight"] = (top,)
    p[f"{a}.group_norm.bias"] = (top,)
    for n in ("to_q", "to_k", "to_v", "to_out.0"):
        p[f"{a}.{n}.weight"] = (top, top)
        p[f"{a}.{n}.bias"] = (top,)
    resnet("decoder.mid_block.resnets.1", top, top)
    for i, j, cin, cout, up in _plan(cfg):
        resnet(f"decoder.up_blocks.{i}.resnets.{j}", cin, cout)
        if up:
            p[f"decoder.up_blocks.{i}.upsamplers.0.conv.weight"] = (cout, cout, 3, 3)
            p[f"decoder.up_blocks.{i}.upsamplers.0.conv.bias"] = (cout,)
    c0 = cfg.block_out_channels[0]
    p.update({"decoder.conv_norm_out.weight": (c0,), "decoder.conv_norm_out.bias": (c0,),
              "decoder.conv_out.weight": (cfg.out_channels, c0, 3, 3),
              "decoder.conv_out.bias": (cfg.out_channels,)})
    return p


def random_param_source(cfg: VaeConfig, seed: int, device, dtype=torch.float32):
    """Parameters drawn on the device: N(0, fan_in^-1/2) weights, N(0, 0.02) biases, GroupNorm
    weights 1 + N(0, 0.1) and biases N(0, 0.1)."""
    import zlib

    shapes = param_shapes(cfg)

    def get(name: str) -> torch.Tensor:
        shp = shapes[name]
        g = torch.Generator(device=device).manual_seed(seed * 1_000_003 + zlib.crc32(name.encode()))
        x = torch.randn(shp, generator=g, device=device, dtype=torch.float32)
        if "norm" in name:
            return 1.0 + 0.1 * x if name.endswith("weight") else 0.1 * x
        x = 0.02 * x if name.endswith("bias") else x * (math.prod(shp[1:]) ** -0.5)
        return x.to(dtype)

    return get


def _ceil(x: int, m: int) -> int:
    return -(-x // m) * m


def pack_conv(w: torch.Tensor, b: torch.Tensor, kq: int, dtype: torch.dtype):
    """A conv weight [Cout, Cin, k, k] as the GEMM operand [Cout padded to 4, k k Cin padded to
    a multiple of kq], taps major and channels minor (the im2col column order), with its bias
    padded alike: (weight, bias, Cout, padded K)."""
    cout, cin, kh, kw = w.shape
    k = kh * kw * cin
    kp, np_ = _ceil(k, kq), _ceil(cout, 4)
    wp = torch.zeros(np_, kp, dtype=torch.float32, device=w.device)
    wp[:cout, :k] = w.permute(0, 2, 3, 1).reshape(cout, k)
    bp = torch.zeros(np_, dtype=torch.float32, device=w.device)
    bp[:cout] = b
    return wp.to(dtype).contiguous(), bp.to(dtype).contiguous(), cout, kp


class VaeDecoder:
    """decode(z [B, latent_channels, h, w] unscaled latents) -> images [B, out_channels, 8 h,
    8 w] in the model dtype (bf16 or fp32)."""

    def __init__(self, cfg: VaeConfig, param_source: Callable[[str], torch.Tensor], *,
                 dtype: torch.dtype = torch.bfloat16, device="cuda"):
        if dtype not in (torch.bfloat16, torch.float32):
            raise NotImplementedError(f"VaeDecoder runs bf16 or fp32, not {dtype}")
        if cfg.use_post_quant_conv:
            raise NotImplementedError("post_quant_conv is not implemented (FLUX.1's VAE has none)")
        for c in cfg.block_out_channels:
            if c % cfg.norm_num_groups or c % 8:
                raise NotImplementedError(f"{c} channels: multiples of 8 and of the groups only")
        self.cfg, self.dtype, self.device = cfg, dtype, torch.device(device)
        self.kq = 64 if dtype == torch.bfloat16 else 4  # the GEMM's K multiple
        self.groups = cfg.norm_num_groups
        shapes = param_shapes(cfg)

        def get(name, dt=None):
            return param_source(name).to(device=self.device, dtype=dt or dtype).contiguous()

        self.conv = {}   # name -> (weight [Np, Kp] in dtype, bias [Np] or None, cout, kpad)
        self.norm = {}   # name -> (weight, bias) fp32
        self.lin = {}    # name -> (weight [N, K], bias [N])
        for name in shapes:
            if not name.endswith(".weight"):
                continue
            base = name[: -len(".weight")]
            if "norm" in base:
                self.norm[base] = (get(name, torch.float32), get(base + ".bias", torch.float32))
            elif len(shapes[name]) == 4:
                self.conv[base] = self._pack_conv(get(name, torch.float32), get(base + ".bias", torch.float32))
        a = "decoder.mid_block.attentions.0"
        self.lin["qkv"] = (torch.cat([get(f"{a}.{n}.weight") for n in ("to_q", "to_k", "to_v")]),
                           torch.cat([get(f"{a}.{n}.bias") for n in ("to_q", "to_k", "to_v")]))
        self.lin["out"] = (get(f"{a}.to_out.0.weight"), get(f"{a}.to_out.0.bias"))
        top = cfg.block_out_channels[-1]
        self._ones = {c: torch.ones(1, c, dtype=torch.bfloat16, device=self.device)
                      for c in set(cfg.block_out_channels) | {_ceil(cfg.out_channels, 4),
                                                              _ceil(top, 4)}}

    def _pack_conv(self, w: torch.Tensor, b: torch.Tensor):
        return pack_conv(w, b, self.kq, self.dtype)

    # ------------------------------------------------------------------ pieces
    def _gemm(self, a, w, bias, out, residual=None):
        if self.dtype == torch.float32:
            kernels.gemm_f32(a, w, bias, residual=residual, out=out)
            return out
        if residual is None:
            p, epi = kernels.Problem(a, w, out, bias), _lib.EPI_NONE
        else:
            p = kernels.Problem(a, w, out, bias, gate=self._ones_for(w.shape[0]), residual=residual)
            epi = _lib.EPI_GATE_RESIDUAL
        kernels.gemm_grouped([p], kind="bf16", epilogue=epi, workspace="shared")
        return out

    def _ones_for(self, n):
        t = self._ones.get(n)
        if t is None:
            t = self._ones[n] = torch.ones(1, n, dtype=torch.bfloat16, device=self.device)
        return t

    def _conv3x3(self, x, hw, name, *, upsample=False, residual=None, out=None):
        """x [H * W, Cin] -> [Ho * Wo, Cout padded to 4]."""
        w, b, _, _ = self.conv[name]
        h, wd = hw
        total = (h * wd) << (2 * int(upsample))
        y = out if out is not None else torch.empty(total, w.shape[0], dtype=self.dtype,
                                                     device=self.device)
        # one implicit GEMM: a one-frame (1, 3, 3) convolution
        kernels.conv_causal(x.contiguous(), hw, x.shape[1], 1, w, b, kt=1, ks=3,
                            upsample=upsample, residual=residual, out=y)
        return y

    def _gn(self, x, name, silu):
        w, b = self.norm[name]
        return kernels.group_norm(x.unsqueeze(0), self.groups, w, b, EPS, silu=silu).squeeze(0)

    def _resnet(self, x, hw, pre):
        h = self._gn(x, f"{pre}.norm1", True)
        h = self._conv3x3(h, hw, f"{pre}.conv1")
        h = self._gn(h, f"{pre}.norm2", True)
        sc = x
        if f"{pre}.conv_shortcut" in self.conv:
            w, b, _, _ = self.conv[f"{pre}.conv_shortcut"]
            sc = self._gemm(x, w, b, torch.empty(x.shape[0], w.shape[0], dtype=self.dtype,
                                                 device=self.device))
        return self._conv3x3(h, hw, f"{pre}.conv2", residual=sc, out=sc if sc is not x else None)

    def _attention(self, x):
        """x [P, C]: x + to_out(softmax(q k^T / sqrt(C)) v) over GroupNorm(x)."""
        pix, c = x.shape
        n = self._gn(x, "decoder.mid_block.attentions.0.group_norm", False)
        wqkv, bqkv = self.lin["qkv"]
        qkv = self._gemm(n, wqkv, bqkv, torch.empty(pix, 3 * c, dtype=self.dtype, device=self.device))
        q, k = qkv[:, :c], qkv[:, c:2 * c]
        if self.dtype == torch.bfloat16 and c % 64 == 0:
            s = kernels.gemm_bf16_f32out(q, k)  # fp32 scores from the bf16 matrix cores
        else:
            if self.dtype != torch.float32:
                q, k = q.float(), k.float()
            s = kernels.gemm_f32(q, k)
        # P V: K = pixels, zero-padded to the GEMM's K multiple when it is not one
        kp = _ceil(pix, self.kq)
        alloc = torch.empty if kp == pix else torch.zeros
        p = alloc(pix, kp, dtype=self.dtype, device=self.device)
        kernels.softmax_rows(s, 1.0 / math.sqrt(c), dtype=self.dtype, out=p[:, :pix])
        del s
        vt = alloc(c, kp, dtype=self.dtype, device=self.device)
        vt[:, :pix] = qkv[:, 2 * c:].t()
        o = self._gemm(p, vt, None, torch.empty(pix, c, dtype=self.dtype, device=self.device))
        del p
        wo, bo = self.lin["out"]
        return self._gemm(o, wo, bo, torch.empty_like(x), residual=x)

    # ------------------------------------------------------------------ decode
    def decode(self, z: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        if z.dim() != 4 or z.shape[1] != cfg.latent_channels:
            raise ValueError(f"z must be [batch, {cfg.latent_channels}, h, w]")
        outs = [self._decode_one(z[i]) for i in range(z.shape[0])]
        return torch.stack(outs)

    __call__ = decode

    def unscale(self, latents: torch.Tensor) -> torch.Tensor:
        """latents / scaling_factor + shift_factor (difflet/models/flux/pipeline.py:448), the
        input decode expects."""
        return latents / self.cfg.scaling_factor + self.cfg.shift_factor

    def _decode_one(self, z):
        cfg = self.cfg
        _, h, w = z.shape
        x = z.to(device=self.device, dtype=self.dtype).permute(1, 2, 0).contiguous().view(h * w, -1)
        hw = (h, w)
        x = self._conv3x3(x, hw, "decoder.conv_in")
        x = self._resnet(x, hw, "decoder.mid_block.resnets.0")
        x = self._attention(x)
        x = self._resnet(x, hw, "decoder.mid_block.resnets.1")
        for i, j, _, _, up in _plan(cfg):
            x = self._resnet(x, hw, f"decoder.up_blocks.{i}.resnets.{j}")
            if up:
                x = self._conv3x3(x, hw, f"decoder.up_blocks.{i}.upsamplers.0.conv", upsample=True)
                hw = (hw[0] * 2, hw[1] * 2)
        x = self._gn(x, "decoder.conv_norm_out", True)
        y = self._conv3x3(x, hw, "decoder.conv_out")[:, : cfg.out_channels]
        return y.reshape(hw[0], hw[1], cfg.out_channels).permute(2, 0, 1).contiguous()
