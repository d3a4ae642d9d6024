"""Rotary tables of the DiT models, computed once per shape on the host in float64 and kept on
the device as fp32 [S, head_dim] cos / sin (the kernels read them per row).

FLUX: FluxPosEmbed (difflet/layers/embeddings.py:148-176) with get_1d_rotary_pos_embed
(:178-244, float64 frequencies, repeat-interleaved) over ids (0, 0, 0) for text tokens and
(0, i, j) for image patch (i, j), text first.

Qwen-Image: the QwenEmbedRope table diffusers' QwenImageTransformer2DModel builds (the
reference converts its complex form to this real one, difflet/models/qwen_image/
modeling_qwen_image.py:46-49,643-651): axes (16, 56, 56), theta 10000, angles in fp32; with
scale_rope the image height / width positions run -(n - n // 2) .. n // 2 - 1 (frame 0), and
text token j takes position max(h // 2, w // 2) + j on all three axes; text first.
"""

from __future__ import annotations

import torch


def _axis(dim: int, pos: torch.Tensor, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64)[: dim // 2] / dim))
    ang = torch.outer(pos.to(torch.float64), freqs)
    return ang.cos().repeat_interleave(2, dim=1), ang.sin().repeat_interleave(2, dim=1)


def flux_ids(txt_len: int, img_hw: tuple[int, int]) -> torch.Tensor:
    h, w = img_hw
    ii, jj = torch.meshgrid(torch.arange(h), torch.arange(w), indexing="ij")
    img = torch.stack([torch.zeros_like(ii), ii, jj], dim=-1).reshape(h * w, 3)
    return torch.cat([torch.zeros(txt_len, 3, dtype=img.dtype), img], dim=0)


def flux_rope_tables(txt_len: int, img_hw: tuple[int, int], axes=(16, 56, 56),
                     device="cuda", theta: float = 10000.0):
    ids = flux_ids(txt_len, img_hw)
    cos, sin = zip(*[_axis(d, ids[:, i], theta) for i, d in enumerate(axes)])
    cos = torch.cat(cos, dim=-1).to(torch.float32)
    sin = torch.cat(sin, dim=-1).to(torch.float32)
    return cos.to(device).contiguous(), sin.to(device).contiguous()


def _qwen_axis(pos: torch.Tensor, dim: int, theta: float) -> torch.Tensor:
    inv = 1.0 / torch.pow(torch.tensor(float(theta)),
                          torch.arange(0, dim, 2, dtype=torch.float32).div(dim))
    return torch.outer(pos.to(torch.float32), inv)


def _centred(n: int) -> torch.Tensor:
    return torch.cat([torch.arange(-(n - n // 2), 0), torch.arange(0, n // 2)])


def qwen_rope_tables(txt_len: int, img_hw: tuple[int, int], axes=(16, 56, 56),
                     device="cuda", theta: float = 10000.0):
    h, w = img_hw
    a0, a1, a2 = axes
    hh, ww = torch.meshgrid(_centred(h), _centred(w), indexing="ij")
    img = torch.cat([_qwen_axis(torch.zeros(h * w), a0, theta),
                     _qwen_axis(hh.reshape(-1), a1, theta),
                     _qwen_axis(ww.reshape(-1), a2, theta)], dim=1)
    start = max(h // 2, w // 2)
    p = torch.arange(start, start + txt_len)
    txt = torch.cat([_qwen_axis(p, a0, theta), _qwen_axis(p, a1, theta),
                     _qwen_axis(p, a2, theta)], dim=1)
    ang = torch.cat([txt, img], dim=0)
    cos = torch.cos(ang).repeat_interleave(2, dim=-1)
    sin = torch.sin(ang).repeat_interleave(2, dim=-1)
    return cos.to(device).contiguous(), sin.to(device).contiguous()


def wan_rope_tables(grid: tuple[int, int, int], head_dim: int = 128, max_seq_len: int = 1024,
                    device="cuda", theta: float = 10000.0):
    """WanRotaryPosEmbed (difflet/models/wan/modeling_wan.py:209-296): axes of head_dim - 2 hw,
    hw, hw dims (hw = 2 * (head_dim // 6)) over (frame, row, column) of the patch grid,
    frame-major; float64 frequencies, repeat-interleaved, fp32 [F * H * W, head_dim]."""
    f, h, w = grid
    hw = 2 * (head_dim // 6)
    dims = (head_dim - 2 * hw, hw, hw)
    ff, yy, xx = torch.meshgrid(torch.arange(f), torch.arange(h), torch.arange(w), indexing="ij")
    cos, sin = [], []
    for d, pos in zip(dims, (ff.reshape(-1), yy.reshape(-1), xx.reshape(-1))):
        freqs = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64)[: d // 2] / d))
        table = torch.outer(torch.arange(max_seq_len, dtype=torch.float64), freqs)
        cos.append(table.cos().repeat_interleave(2, dim=1).float()[pos])
        sin.append(table.sin().repeat_interleave(2, dim=1).float()[pos])
    return (torch.cat(cos, dim=1).to(device).contiguous(),
            torch.cat(sin, dim=1).to(device).contiguous())
