"""Rotary embeddings for the rocm backend on the HIP rope kernel.

apply_rotary_emb      -- the stride-2 law of difflet/backends/cpu/ops_impl/embeddings.py:6-14
                         (cos of the even table entries, sin of the odd ones);
apply_rotary_emb_fp32 -- diffusers' interleaved law of
                         difflet/backends/_torch_megatron/embeddings.py:24-33.
Both compute in fp32 and round once to the input dtype (the stride-2 reference rounds after
each product in the input dtype; for fp32 inputs the two agree to fp32 rounding).

Tables broadcast against the input with one position axis: [..., S, D] shaped tables (leading
dims 1) against an input whose position axis is the table's S axis. The kernel reads the
table per position; inputs whose position axis is not the second to last are viewed so.
"""

from __future__ import annotations

import torch

from difflet_amd.backends.rocm.ops_impl import library


def _table(t, x, pos):
    """A table broadcastable to x as fp32 [S, D] along x's position axis `pos`."""
    nd = x.dim()
    t = torch.as_tensor(t, device=x.device)
    t = t.reshape((1,) * (nd - t.dim()) + tuple(t.shape)).movedim(pos, -2)
    t = t.reshape(-1, x.shape[-1]).to(torch.float32)
    return t.expand(x.shape[pos], -1).contiguous() if t.shape[0] == 1 else t.contiguous()


def _rope(x, cos, sin, law: int):
    if x.device.type != "cuda":
        raise ValueError(f"rocm rotary embedding takes device tensors, got one on {x.device}")
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise NotImplementedError(f"rocm rotary embedding: unsupported dtype {x.dtype}")
    nd = x.dim()
    shapes = [tuple(torch.as_tensor(t).shape) for t in (cos, sin)]
    varying = sorted({nd - len(sh) + i for sh in shapes for i, n in enumerate(sh[:-1])
                      if n != 1 and nd - len(sh) + i < nd - 1})
    if len(varying) > 1:
        raise NotImplementedError("rocm rotary embedding: tables may vary along one position axis")
    pos = varying[0] if varying else nd - 2
    c, sn = _table(cos, x, pos), _table(sin, x, pos)
    if c.shape[0] != x.shape[pos]:
        raise ValueError(f"rotary table length {c.shape[0]} does not match the input's "
                         f"{x.shape[pos]} positions")
    y = library.rope(x.movedim(pos, -2).contiguous(), c, sn, law)
    return y.movedim(-2, pos).contiguous() if pos != nd - 2 else y


def apply_rotary_emb(hidden_states, freqs_cos, freqs_sin):
    return _rope(hidden_states, freqs_cos, freqs_sin, law=1)


def apply_rotary_emb_fp32(hidden_states, freqs_cos, freqs_sin):
    return _rope(hidden_states, freqs_cos, freqs_sin, law=0)


__all__ = ["apply_rotary_emb", "apply_rotary_emb_fp32"]
