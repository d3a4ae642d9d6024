"""Wan's 3D causal VAE decoder on the gfx950 kernels: WanVAEDecoderModel
(difflet/models/wan/vae/modeling_vae.py:509-560), the decoder-only restatement of diffusers'
AutoencoderKLWan that the CUDA flow calls as ``vae.decode`` in the model dtype
(difflet/backends/cuda/wan/application.py:115-134), after the pipeline's ``latents * std + mean``
(difflet/models/wan/pipeline.py:544-554). Qwen-Image's VAE is the same decoder on one latent
frame (difflet/models/wan/vae/regions.py:3-6). bf16 or fp32.

The decode walks the latent video one frame (a chunk) at a time, as the reference does: chunk 0
decodes to one frame, every later chunk to 2^u frames (u temporal upsamplings). Activations are
channels-last frames, [frames][pixels][channels]. Each causal 3x3x3 convolution is one implicit
GEMM (kernels.conv_causal: the im2col rows gathered into the matrix kernel's LDS, never written)
over the chunk's frames and a two-frame cache of the convolution's own input from the chunks
before (zeros at the start, the reference's front padding), passed as two frames in front of
the chunk's, with the weight repacked [Cout][dt][ky][kx][Cin] once at load; the cache then takes
the last two frames of (cache, chunk). The time convolution of an upsample3d resampler is a (3, 1, 1) causal
convolution that skips chunk 0 (the reference's "Rep"); its [t][pixels][2C] output is read as
the interleaved frames 2t, 2t + 1 by the resampler's convolution, with the nearest 2x upsampling
of that 3x3 Conv2d folded into its addressing. WanRMSNorm (+ SiLU) is one row kernel.
The mid block's attention (one head over a frame's pixels with all channels) runs as GEMMs:
fp32 scores, the row softmax kernel, P V, then the output projection with the residual.
"""

from __future__ import annotations

import dataclasses
import math
import zlib
from typing import Callable, Optional

import torch

from difflet_amd import _lib, kernels

EPS = 1e-12             # F.normalize's eps in WanRMSNorm


@dataclasses.dataclass(frozen=True)
class WanVaeConfig:
    """WanVAEDecoderConfig (modeling_vae.py:43-89): the same fields, defaults (Wan 2.1 / 2.2's
    VAE) and refusals."""

    base_dim: int = 96
    decoder_base_dim: Optional[int] = None
    z_dim: int = 16
    dim_mult: tuple = (1, 2, 4, 4)
    num_res_blocks: int = 2
    attn_scales: tuple = ()
    temperal_downsample: tuple = (False, True, True)
    dropout: float = 0.0
    latents_mean: tuple = ()
    latents_std: tuple = ()
    is_residual: bool = False
    in_channels: int = 3
    out_channels: int = 3
    patch_size: Optional[int] = None
    scale_factor_temporal: int = 4
    scale_factor_spatial: int = 8

    def __post_init__(self):
        if self.decoder_base_dim is None:
            object.__setattr__(self, "decoder_base_dim", self.base_dim)
        for f in ("dim_mult", "attn_scales", "temperal_downsample", "latents_mean", "latents_std"):
            object.__setattr__(self, f, tuple(getattr(self, f)))
        if self.is_residual:
            raise NotImplementedError("the Wan VAE decoder supports only is_residual=False")
        if self.patch_size is not None:
            raise NotImplementedError("the Wan VAE decoder does not support a patchified VAE")
        if self.scale_factor_temporal != 4:
            raise NotImplementedError("the Wan VAE decoder expects temporal scale factor 4")
        if self.scale_factor_spatial != 8:
            raise NotImplementedError("the Wan VAE decoder expects spatial scale factor 8")
        if len(self.dim_mult) < 2:
            raise ValueError("dim_mult must contain at least two stages")
        if len(self.temperal_downsample) != len(self.dim_mult) - 1:
            raise ValueError("temperal_downsample must have len(dim_mult) - 1 entries")
        if self.attn_scales:
            raise NotImplementedError("decoder attention scales are not supported")

    @property
    def temperal_upsample(self) -> tuple:
        return tuple(reversed(self.temperal_downsample))

    @property
    def dims(self) -> list[int]:
        m = list(self.dim_mult)
        return [int(self.decoder_base_dim) * u for u in [m[-1]] + m[::-1]]

    @classmethod
    def from_diffusers_dict(cls, raw: dict) -> "WanVaeConfig":
        """From AutoencoderKLWan's config.json; keys this config does not have are dropped."""
        names = {f.name for f in dataclasses.fields(cls)}
        return cls(**{k: v for k, v in raw.items() if k in names})


WAN_VAE = WanVaeConfig()


def plan(cfg: WanVaeConfig) -> list[tuple[int, int, int, Optional[str]]]:
    """Up blocks: (index, in channels, out channels, resampler mode or None)
    (modeling_vae.py:437-456)."""
    dims, n, out = cfg.dims, len(cfg.dim_mult), []
    for i, (cin, cout) in enumerate(zip(dims[:-1], dims[1:])):
        if i > 0:
            cin //= 2
        mode = None
        if i != n - 1:
            mode = "upsample3d" if cfg.temperal_upsample[i] else "upsample2d"
        out.append((i, cin, cout, mode))
    return out


def param_shapes(cfg: WanVaeConfig) -> dict[str, tuple]:
    """AutoencoderKLWan's decoder and post_quant_conv keys (the reference's state dict)."""
    z, top = cfg.z_dim, cfg.dims[0]
    p = {"post_quant_conv.weight": (z, z, 1, 1, 1), "post_quant_conv.bias": (z,),
         "decoder.conv_in.weight": (top, z, 3, 3, 3), "decoder.conv_in.bias": (top,)}

    def resnet(pre, cin, cout):
        p.update({f"{pre}.norm1.gamma": (cin, 1, 1, 1), f"{pre}.conv1.weight": (cout, cin, 3, 3, 3),
                  f"{pre}.conv1.bias": (cout,), f"{pre}.norm2.gamma": (cout, 1, 1, 1),
                  f"{pre}.conv2.weight": (cout, cout, 3, 3, 3), f"{pre}.conv2.bias": (cout,)})
        if cin != cout:
            p[f"{pre}.conv_shortcut.weight"] = (cout, cin, 1, 1, 1)
            p[f"{pre}.conv_shortcut.bias"] = (cout,)

    resnet("decoder.mid_block.resnets.0", top, top)
    a = "decoder.mid_block.attentions.0"
    p.update({f"{a}.norm.gamma": (top, 1, 1), f"{a}.to_qkv.weight": (3 * top, top, 1, 1),
              f"{a}.to_qkv.bias": (3 * top,), f"{a}.proj.weight": (top, top, 1, 1),
              f"{a}.proj.bias": (top,)})
    resnet("decoder.mid_block.resnets.1", top, top)
    for i, cin, cout, mode in plan(cfg):
        c = cin
        for j in range(cfg.num_res_blocks + 1):
            resnet(f"decoder.up_blocks.{i}.resnets.{j}", c, cout)
            c = cout
        if mode is not None:
            u = f"decoder.up_blocks.{i}.upsamplers.0"
            p[f"{u}.resample.1.weight"] = (cout // 2, cout, 3, 3)
            p[f"{u}.resample.1.bias"] = (cout // 2,)
            if mode == "upsample3d":
                p[f"{u}.time_conv.weight"] = (2 * cout, cout, 3, 1, 1)
                p[f"{u}.time_conv.bias"] = (2 * cout,)
    last = cfg.dims[-1]
    p.update({"decoder.norm_out.gamma": (last, 1, 1, 1),
              "decoder.conv_out.weight": (cfg.out_channels, last, 3, 3, 3),
              "decoder.conv_out.bias": (cfg.out_channels,)})
    return p


def random_param_source(cfg: WanVaeConfig, seed: int, device, dtype=torch.float32):
    """Parameters drawn on the device: N(0, fan_in^-1/2) convolutions, N(0, 0.02) biases, RMS
    norm gammas 1 + N(0, 0.1)."""
    shapes = param_shapes(cfg)

    def get(name: str) -> torch.Tensor:
        shp = shapes[name]
        g = torch.Generator(device=device).manual_seed(seed * 1_000_003 + zlib.crc32(name.encode()))
        x = torch.randn(shp, generator=g, device=device, dtype=torch.float32)
        if name.endswith("gamma"):
            return 1.0 + 0.1 * x
        x = 0.02 * x if name.endswith("bias") else x * (math.prod(shp[1:]) ** -0.5)
        return x.to(dtype)

    return get


def _ceil(x: int, m: int) -> int:
    return -(-x // m) * m


@dataclasses.dataclass
class _Conv:
    """A convolution as a GEMM operand: weight [Cout padded to 4, K padded to kq] with columns
    (dt, ky, kx, cin), bias padded alike."""
    w: torch.Tensor
    b: torch.Tensor
    cout: int
    cin: int
    kt: int
    ks: int
    kpad: int


def pack_conv(w: torch.Tensor, b: torch.Tensor, kq: int, dtype: torch.dtype) -> _Conv:
    """A Conv3d weight [Cout, Cin, kt, ks, ks] or Conv2d weight [Cout, Cin, ks, ks] (kt = 1) as
    the im2col GEMM's weight operand."""
    if w.dim() == 4:
        w = w.unsqueeze(2)
    cout, cin, kt, kh, kw = w.shape
    if kh != kw:
        raise NotImplementedError("square spatial kernels only")
    k = kt * kh * kw * cin
    kp, np_ = _ceil(k, kq), _ceil(cout, 4)
    wp = torch.zeros(np_, kp, dtype=torch.float32, device=w.device)
    wp[:cout, :k] = w.permute(0, 2, 3, 4, 1).reshape(cout, k)
    bp = torch.zeros(np_, dtype=torch.float32, device=w.device)
    bp[:cout] = b
    return _Conv(wp.to(dtype).contiguous(), bp.to(dtype).contiguous(), cout, cin, kt, kh, kp)


class _Chunk:
    """Frames of one chunk at one level: data [frames, pixels, ld] (channels in the first C
    columns of each row), (h, w), C; full: None, or a [2 + frames, pixels, C] buffer whose
    frames 2.. are data, its first two left for a causal convolution's cache."""

    __slots__ = ("data", "frames", "hw", "c", "full")

    def __init__(self, data, frames, hw, c, full=None):
        self.data, self.frames, self.hw, self.c, self.full = data, frames, hw, c, full

    @property
    def rows(self) -> torch.Tensor:
        return self.data.view(self.frames * self.hw[0] * self.hw[1], -1)


class WanVaeDecoder:
    """decode(z [B, z_dim, T, h, w] latents) -> video [B, out_channels, frames, 8 h, 8 w] in the
    model dtype, clamped to [-1, 1]; frames = 1 + (T - 1) 2^u for u temporal upsamplings."""

    def __init__(self, cfg: WanVaeConfig, param_source: Callable[[str], torch.Tensor], *,
                 dtype: torch.dtype = torch.bfloat16, device="cuda"):
        if dtype not in (torch.bfloat16, torch.float32):
            raise NotImplementedError(f"WanVaeDecoder runs bf16 or fp32, not {dtype}")
        halves = {cout // 2 for _, _, cout, mode in plan(cfg) if mode is not None}
        for c in set(cfg.dims) | {cfg.z_dim} | halves:
            if c % 8:
                raise NotImplementedError(f"{c} channels: multiples of 8 only")
        self.cfg, self.dtype, self.device = cfg, dtype, torch.device(device)
        self.kq = 64 if dtype == torch.bfloat16 else 4  # the GEMM's K multiple
        shapes = param_shapes(cfg)

        def get(name, dt=None):
            return param_source(name).to(device=self.device, dtype=dt or torch.float32).contiguous()

        self.conv: dict[str, _Conv] = {}
        self.gamma: dict[str, torch.Tensor] = {}
        for name, shp in shapes.items():
            if name.endswith(".gamma"):
                self.gamma[name[: -len(".gamma")]] = get(name).reshape(-1).contiguous()
            elif name.endswith(".weight"):
                base = name[: -len(".weight")]
                self.conv[base] = pack_conv(get(name), get(base + ".bias"), self.kq, dtype)
        self._ones: dict[int, torch.Tensor] = {}
        self.time_convs = [f"decoder.up_blocks.{i}.upsamplers.0.time_conv"
                           for i, _, _, mode in plan(cfg) if mode == "upsample3d"]

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

    def _conv(self, name: str, x: _Chunk, *, cache: Optional[torch.Tensor] = None,
              upsample: bool = False, frames_per_block: int = 1, residual=None,
              out=None) -> _Chunk:
        """The convolution `name` over the chunk's frames (cache: the two frames before them) as
        one implicit GEMM; the output's rows are padded to Cout rounded up to 4."""
        cv = self.conv[name]
        h, w = x.hw
        up = int(upsample)
        frames = x.frames
        ho, wo = h << up, w << up
        total = frames * ho * wo
        np_ = cv.w.shape[0]
        y = out if out is not None else torch.empty(total, np_, dtype=self.dtype, device=self.device)
        data = x.data
        ld = data.shape[-1]
        if frames_per_block == 2:  # the time convolution's [t][pixels][2C] output as 2t frames
            fs, sub, pstride = h * w * ld, x.c, ld
        else:
            fs, sub, pstride = h * w * ld, 0, ld
        if cv.kt == 1 and cv.ks == 1 and not up and cv.kpad == cv.cin and ld == cv.cin:
            self._gemm(x.rows, cv.w, cv.b, y, residual)   # a 1x1x1 convolution is the GEMM itself
        elif cache is not None:
            # one implicit GEMM; a causal convolution reads its cache as the two frames in front
            if x.full is not None:
                full = x.full
                full[:2].copy_(cache)
            else:
                full = torch.cat([cache, data[:, :, : x.c]])
            kernels.conv_causal(full, (h, w), cv.cin, frames, cv.w, cv.b, kt=cv.kt, ks=cv.ks,
                                upsample=upsample, lead_frames=2, residual=residual, out=y)
        else:
            kernels.conv_causal(data, (h, w), cv.cin, frames, cv.w, cv.b, kt=cv.kt, ks=cv.ks,
                                upsample=upsample, frames_per_block=frames_per_block,
                                frame_stride=fs, sub_stride=sub, pixel_stride=pstride,
                                residual=residual, out=y)
        return _Chunk(y.view(frames, ho * wo, np_), frames, (ho, wo), cv.cout)

    def _cache(self, state: dict, name: str, x: _Chunk) -> torch.Tensor:
        c = state.get(name)
        if c is None:
            c = state[name] = torch.zeros(2, x.hw[0] * x.hw[1], x.c, dtype=self.dtype,
                                          device=self.device)
        return c

    @staticmethod
    def _roll(cache: torch.Tensor, x: _Chunk):
        """cache <- the last two frames of (cache, x) (the reference's _tail_cache rule)."""
        if x.frames >= 2:
            cache.copy_(x.data[x.frames - 2:x.frames, :, : x.c])
        else:
            cache[0].copy_(cache[1])
            cache[1].copy_(x.data[0, :, : x.c])

    def _causal(self, state: dict, name: str, x: _Chunk, **kw) -> _Chunk:
        cache = self._cache(state, name, x)
        y = self._conv(name, x, cache=cache, **kw)
        self._roll(cache, x)
        return y

    def _norm(self, name: str, x: _Chunk, silu: bool, causal: bool = False) -> _Chunk:
        """causal: the output feeds a causal convolution, which reads it with its cache in front
        (frames allocated with two leading ones)."""
        pix = x.hw[0] * x.hw[1]
        lead = 2 if causal else 0
        full = torch.empty(lead + x.frames, pix, x.c, dtype=self.dtype, device=self.device)
        y = kernels.rms_norm_channels(x.rows[:, : x.c], self.gamma[name], eps=EPS, silu=silu,
                                      out=full[lead:].view(-1, x.c))
        return _Chunk(full[lead:], x.frames, x.hw, x.c, full if lead else None)

    def _resnet(self, state: dict, pre: str, x: _Chunk) -> _Chunk:
        sc = x
        if f"{pre}.conv_shortcut" in self.conv:
            sc = self._conv(f"{pre}.conv_shortcut", x)
        h = self._norm(f"{pre}.norm1", x, True, causal=True)
        h = self._causal(state, f"{pre}.conv1", h)
        h = self._norm(f"{pre}.norm2", h, True, causal=True)
        res = sc.rows
        return self._causal(state, f"{pre}.conv2", h, residual=res,
                            out=res if sc is not x else None)

    def _attention(self, pre: str, x: _Chunk) -> _Chunk:
        """Per frame: x + proj(softmax(q k^T / sqrt(C)) v) over RMSNorm(x)."""
        c = x.c
        pix = x.hw[0] * x.hw[1]
        n = self._norm(f"{pre}.norm", x, False)
        out = torch.empty_like(x.rows)
        kp = _ceil(pix, self.kq)
        alloc = torch.empty if kp == pix else torch.zeros
        for f in range(x.frames):
            rows = slice(f * pix, (f + 1) * pix)
            qkv = self._conv(f"{pre}.to_qkv", _Chunk(n.data[f:f + 1], 1, x.hw, c)).rows
            q, k = qkv[:, :c], qkv[:, c:2 * c]
            if self.dtype == torch.bfloat16 and c % 64 == 0:
                s = kernels.gemm_bf16_f32out(q, k)  # fp32 scores from the bf16 matrix cores
            else:
                if self.dtype != torch.float32 or pix % 4:
                    # fp32 scores; the fp32 GEMM's N (keys) padded to a multiple of 4 with zero
                    # keys, whose scores the softmax never reads (cols = pix)
                    kf = torch.zeros(_ceil(pix, 4), c, dtype=torch.float32, device=self.device)
                    kf[:pix] = k
                    q, k = q.float(), kf
                s = kernels.gemm_f32(q, k)
            p = alloc(pix, kp, dtype=self.dtype, device=self.device)
            kernels.softmax_rows(s[:, :pix], 1.0 / math.sqrt(c), dtype=self.dtype, out=p[:, :pix])
            del s
            vt = alloc(c, kp, dtype=self.dtype, device=self.device)
            vt[:, :pix] = qkv[:, 2 * c:].t()
            o = self._gemm(p, vt, None, torch.empty(pix, c, dtype=self.dtype, device=self.device))
            del p, vt
            self._conv(f"{pre}.proj", _Chunk(o.view(1, pix, c), 1, x.hw, c),
                       residual=x.rows[rows], out=out[rows])
        return _Chunk(out.view(x.frames, pix, c), x.frames, x.hw, c)

    def _resample(self, state: dict, pre: str, mode: str, x: _Chunk) -> _Chunk:
        fpb = 1
        if mode == "upsample3d":
            name = f"{pre}.time_conv"
            seen = state.setdefault("_seen", set())
            if name in seen:
                t = self._causal(state, name, x)     # [t][pixels][2C]
                x = _Chunk(t.data, 2 * x.frames, x.hw, x.c)
                fpb = 2
            else:
                seen.add(name)                       # chunk 0: the reference's "Rep"
        return self._conv(f"{pre}.resample.1", x, upsample=True, frames_per_block=fpb)

    # ------------------------------------------------------------------ decode
    def denormalize(self, latents: torch.Tensor) -> torch.Tensor:
        """latents * std + mean per channel when the config has both (pipeline.py:544-554)."""
        mean, std = self.cfg.latents_mean, self.cfg.latents_std
        if not mean or not std:
            return latents
        m = torch.tensor(mean, dtype=latents.dtype, device=latents.device).view(1, -1, 1, 1, 1)
        s = torch.tensor(std, dtype=latents.dtype, device=latents.device).view(1, -1, 1, 1, 1)
        return latents * s + m

    def decode(self, z: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        if z.dim() != 5 or z.shape[1] != cfg.z_dim:
            raise ValueError(f"z must be [batch, {cfg.z_dim}, frames, h, w]")
        return torch.stack([self._decode_one(z[i]) for i in range(z.shape[0])])

    __call__ = decode

    def _decode_one(self, z: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        zc, t, h, w = z.shape
        x = z.to(device=self.device, dtype=self.dtype).permute(1, 2, 3, 0).contiguous()
        x = self._conv("post_quant_conv", _Chunk(x.view(t, h * w, zc), t, (h, w), zc))
        state: dict = {}
        frames = []
        for i in range(t):
            c0 = _Chunk(x.data[i:i + 1].contiguous(), 1, (h, w), x.c)
            frames.append(self._decode_chunk(state, c0))
        n_frames = sum(f.frames for f in frames)
        ho, wo = frames[0].hw
        video = torch.empty(cfg.out_channels, n_frames, ho, wo, dtype=self.dtype, device=self.device)
        f0 = 0
        flat = video.view(cfg.out_channels, -1)
        for f in frames:
            n = f.frames * ho * wo
            plane = kernels.rows_to_planes(f.rows, cfg.out_channels, lo=-1.0, hi=1.0)
            flat[:, f0:f0 + n].copy_(plane)
            f0 += n
        return video

    def _decode_chunk(self, state: dict, x: _Chunk) -> _Chunk:
        cfg = self.cfg
        x = self._causal(state, "decoder.conv_in", x)
        x = self._resnet(state, "decoder.mid_block.resnets.0", x)
        x = self._attention("decoder.mid_block.attentions.0", x)
        x = self._resnet(state, "decoder.mid_block.resnets.1", x)
        for i, _, _, mode in plan(cfg):
            for j in range(cfg.num_res_blocks + 1):
                x = self._resnet(state, f"decoder.up_blocks.{i}.resnets.{j}", x)
            if mode is not None:
                x = self._resample(state, f"decoder.up_blocks.{i}.upsamplers.0", mode, x)
        x = self._norm("decoder.norm_out", x, True, causal=True)
        return self._causal(state, "decoder.conv_out", x)
