"""Rotary tables of the DiT models, computed once per shape on the host in float64 and kept on
the device as fp32 [S, head_dim] cos / sin (the kernels read them per row).

FLUX: FluxPosEmbed (difflet/layers/embeddings.py:148-176) with get_1d_rotary_pos_embed
(:178-244, float64 frequencies, repeat-interleaved) over ids (0, 0, 0) for text tokens and
(0, i, j) for image patch (i, j), text first.
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
