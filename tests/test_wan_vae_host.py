"""The Wan VAE decoder's host walk (difflet_amd/vae/wan.py) on the CPU: chunking, the two-frame
caches, the skipped first time convolution, the interleaved-frame strides and the row ranges,
with every device kernel replaced by a torch statement of its C-ABI contract
(include/difflet_rocm.h). The decode then equals the oracle (oracle/wan_vae.py); the kernels
themselves are checked on the GPU (tests/test_gpu_wan_vae.py)."""

import pytest
import torch
import torch.nn.functional as F

from difflet_amd import _lib, kernels
from difflet_amd.vae import wan as dwan
from oracle import wan_vae as ow


def rel_l2(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def _im2col_causal(x, hw, channels, *, kt, ks, kpad, upsample=False, cache=None,
                   frames_per_block=1, frame_stride=None, sub_stride=0, pixel_stride=None,
                   row0=0, rows=None, out=None):
    h, w = hw
    pix, ld = h * w, channels if pixel_stride is None else pixel_stride
    fs = pix * ld if frame_stride is None else frame_stride
    up = 2 if upsample else 1
    po = pix * up * up
    if rows is None:
        rows = (x.numel() // (pix * ld)) * po - row0
    last = (row0 + rows - 1) // po
    flat = x.reshape(-1)
    frames = []
    for f in range(last + 1):
        base = (f // frames_per_block) * fs + (f % frames_per_block) * sub_stride
        idx = base + torch.arange(pix)[:, None] * ld + torch.arange(channels)[None]
        frames.append(flat[idx])
    prev = (torch.zeros(2, pix, channels, dtype=x.dtype) if cache is None else cache)
    seq = torch.cat([prev, torch.stack(frames)])          # [2 + F, pix, C]
    img = seq.view(-1, h, w, channels).permute(0, 3, 1, 2).float()
    if upsample:
        img = F.interpolate(img, scale_factor=2.0, mode="nearest")
    ho, wo = img.shape[2:]
    p = ks // 2
    img = F.pad(img, (p, p, p, p))
    out_rows = []
    for t in range(last + 1):
        taps = [img[2 + t + dt - (kt - 1), :, ky:ky + ho, kx:kx + wo]
                for dt in range(kt) for ky in range(ks) for kx in range(ks)]
        out_rows.append(torch.stack(taps, 0).permute(2, 3, 0, 1).reshape(ho * wo, -1))
    a = torch.cat(out_rows)[row0:row0 + rows]
    return F.pad(a, (0, kpad - a.shape[1])).to(x.dtype)


def _conv_causal(x, hw, channels, frames, w, bias=None, *, kt, ks, upsample=False,
                 lead_frames=0, frames_per_block=1, frame_stride=None, sub_stride=0,
                 pixel_stride=None, residual=None, out=None):
    """The contract of kernels.conv_causal: the im2col rows of the chunk's frames (buffer frames
    lead_frames.. of x; the ones in front are frames -lead_frames..-1, zeros before) times w."""
    h, wd = hw
    pix = h * wd
    ld = channels if pixel_stride is None else pixel_stride
    fs = pix * ld if frame_stride is None else frame_stride
    flat = x.reshape(-1)

    def frame(b):
        base = (b // frames_per_block) * fs + (b % frames_per_block) * sub_stride
        return flat[base + torch.arange(pix)[:, None] * ld + torch.arange(channels)[None]]

    seq = torch.stack([frame(b) for b in range(lead_frames + frames)])
    cache = torch.cat([torch.zeros(2 - lead_frames, pix, channels, dtype=x.dtype),
                       seq[:lead_frames]])
    cols = _im2col_causal(seq[lead_frames:].contiguous(), hw, channels, kt=kt, ks=ks,
                          kpad=w.shape[1], upsample=upsample, cache=cache)
    acc = cols.float() @ w.float().t()
    acc = acc + (0 if bias is None else bias.float())
    acc = acc + (0 if residual is None else residual[:, : w.shape[0]].float())
    if out is None:
        return acc.to(x.dtype)
    out[:, : w.shape[0]].copy_(acc)
    return out


def _rms(x, gamma, *, eps=1e-12, silu=False, out=None):
    c = x.shape[1]
    y = x.float() * (c ** 0.5) / x.float().norm(dim=1, keepdim=True).clamp_min(eps) * gamma
    y = F.silu(y) if silu else y
    if out is None:
        return y.to(x.dtype)
    out.copy_(y)
    return out


def _planes(x, channels, *, lo=float("-inf"), hi=float("inf"), out=None):
    return x[:, :channels].t().clamp(lo, hi).contiguous()


def _gemm_grouped(problems, *, kind="bf16", epilogue=_lib.EPI_NONE, workspace=None, **kw):
    for p in problems:
        acc = p.a.float() @ p.w.float().t()
        if p.bias is not None:
            acc = acc + p.bias.float()
        if epilogue == _lib.EPI_GATE_RESIDUAL:
            acc = p.gate.float() * acc + p.residual.float()
        p.c.copy_(acc)


def _gemm_f32(a, w, bias=None, *, residual=None, out=None):
    if a.shape[1] % 4 or w.shape[0] % 4:
        raise ValueError("gemm_f32: K and N must be multiples of 4")
    acc = a @ w.t() + (0 if bias is None else bias)
    acc = acc + (0 if residual is None else residual)
    if out is None:
        return acc
    out.copy_(acc)
    return out


def _softmax(s, scale, *, dtype=torch.float32, out=None):
    if s.stride(1) != 1:
        raise ValueError("softmax_rows: rows must be contiguous")
    p = torch.softmax(s * scale, dim=-1).to(dtype)
    if out is None:
        return p
    out.copy_(p)
    return out


@pytest.fixture
def cpu_kernels(monkeypatch):
    monkeypatch.setattr(kernels, "im2col_causal", _im2col_causal)
    monkeypatch.setattr(kernels, "conv_causal", _conv_causal)
    monkeypatch.setattr(kernels, "rms_norm_channels", _rms)
    monkeypatch.setattr(kernels, "rows_to_planes", _planes)
    monkeypatch.setattr(kernels, "gemm_grouped", _gemm_grouped)
    monkeypatch.setattr(kernels, "gemm_f32", _gemm_f32)
    monkeypatch.setattr(kernels, "softmax_rows", _softmax)


SMALL = ow.WanVaeShape(base_dim=8, z_dim=16, dim_mult=(1, 2, 4, 4), num_res_blocks=1,
                       temperal_downsample=(False, True, True))


def _cfg(shape):
    return dwan.WanVaeConfig(base_dim=shape.base_dim, z_dim=shape.z_dim, dim_mult=shape.dim_mult,
                             num_res_blocks=shape.num_res_blocks,
                             temperal_downsample=shape.temperal_downsample)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_host_walk_equals_the_oracle(cpu_kernels, monkeypatch, dtype):
    """Three latent frames (two temporal upsamplings), a 3 x 5 latent; every convolution one
    implicit GEMM, a causal one's cache passed as the two frames in front of the chunk's."""
    store = None if dtype == torch.float32 else dtype
    w = ow.weights(SMALL, 5, store)
    dec = dwan.WanVaeDecoder(_cfg(SMALL), lambda n: w[n], dtype=dtype, device="cpu")
    z = torch.randn(1, SMALL.z_dim, 3, 3, 5, generator=torch.Generator().manual_seed(6))
    ref = ow.decode(w, SMALL, z, store=store)
    out = dec.decode(z)
    assert out.dtype == dtype and tuple(out.shape) == tuple(ref.shape) == (1, 3, 9, 24, 40)
    assert rel_l2(out, ref) < (1e-5 if dtype == torch.float32 else 2e-2)


def test_decoder_refuses_what_it_cannot_run():
    with pytest.raises(NotImplementedError):
        dwan.WanVaeDecoder(dwan.WAN_VAE, lambda n: None, dtype=torch.float16, device="cpu")
    with pytest.raises(NotImplementedError, match="multiples of 8"):
        dwan.WanVaeDecoder(dwan.WanVaeConfig(base_dim=6), lambda n: None, device="cpu")
