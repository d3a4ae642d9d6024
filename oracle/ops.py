"""CPU restatement of the reference op semantics (fp32 torch on the CPU). Test infrastructure
only (see oracle/__init__.py)."""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def attention(q, k, v, *, scale=None, causal=False, attention_mask=None, bound_min=None,
              bound_max=None):
    """difflet/backends/cpu/ops_impl/attention.py:8-48: scores in the input dtype, masked with
    finfo(dtype).min, softmax in fp32, probabilities cast to v's dtype, then @ v."""
    if bound_min is not None or bound_max is not None:
        if bound_min is None or bound_max is None:
            raise ValueError("bound_min and bound_max must both be provided")
        if attention_mask is not None:
            raise ValueError("attention_mask and bounds are mutually exclusive")
        key_idx = torch.arange(k.shape[-2]).view(1, 1, -1)
        attention_mask = (key_idx >= bound_min) & (key_idx < bound_max)
    scale = 1.0 if scale is None else scale
    scores = torch.matmul(q, k.transpose(-1, -2)) * scale
    if causal:
        ql, kl = scores.shape[-2:]
        tri = torch.ones((ql, kl), dtype=torch.bool).tril()
        scores = scores.masked_fill(~tri, torch.finfo(scores.dtype).min)
    if attention_mask is not None:
        if attention_mask.dtype == torch.bool:
            scores = scores.masked_fill(~attention_mask, torch.finfo(scores.dtype).min)
        else:
            scores = scores + attention_mask.to(scores.dtype)
    probs = torch.softmax(scores.float(), dim=-1).to(v.dtype)
    return torch.matmul(probs, v)


def rounder(dtype=None):
    """Identity, or a round trip through ``dtype`` (returned in fp32): the oracle blocks apply it
    wherever a device that stores its activations in ``dtype`` rounds them, so a quantized
    linear downstream sees the same inputs on both sides."""
    if dtype is None:
        return lambda x: x
    return lambda x: x.to(dtype).float()


def rms_norm_cpu_law(x, weight, eps):
    """difflet/backends/cpu/ops_impl/norm.py:19-22: fp32 variance, cast to x's dtype before
    +eps, normalise and apply the weight in x's dtype."""
    variance = x.to(torch.float32).pow(2).mean(dim=-1, keepdim=True)
    y = x * torch.rsqrt(variance.to(x.dtype) + eps)
    return y * weight


def rms_norm_fp32(x, weight, eps):
    """difflet/backends/_torch_megatron/norm.py:35-45: fp32 statistics, normalisation and
    affine, one cast back."""
    sq = x.float().pow(2).sum(dim=-1, keepdim=True)
    y = x.float() * torch.rsqrt(sq / x.shape[-1] + eps)
    if weight is not None:
        y = y * weight.float()
    return y.to(x.dtype)


def apply_rotary_emb(x, cos, sin):
    """difflet/backends/cpu/ops_impl/embeddings.py:6-14 (the stride-2 law, input dtype)."""
    x1, x2 = x.unflatten(-1, (-1, 2)).unbind(-1)
    c = cos[..., 0::2]
    s = sin[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x1 * c - x2 * s
    out[..., 1::2] = x1 * s + x2 * c
    return out.to(x.dtype)


def apply_rotary_emb_fp32(x, cos, sin):
    """difflet/backends/_torch_megatron/embeddings.py:24-33 (interleaved pairs in fp32)."""
    xr, xi = x.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    rot = torch.stack([-xi, xr], dim=-1).flatten(-2)
    return (x.float() * cos + rot.float() * sin).to(x.dtype)


def layer_norm(x, eps=1e-6):
    """nn.LayerNorm(dim, elementwise_affine=False, eps) (difflet/backends/cpu/ops_impl/norm.py:9)."""
    return F.layer_norm(x, (x.shape[-1],), eps=eps)


def ada_modulate(x, shift, scale, eps=1e-6):
    """LN(x) * (1 + scale) + shift, scale/shift [B, D] broadcast over tokens
    (difflet/layers/normalization.py:83,146)."""
    return layer_norm(x, eps) * (1 + scale[:, None]) + shift[:, None]


def gelu_tanh(x):
    """difflet/layers/activations.py:59-65 (approximate='tanh')."""
    return F.gelu(x, approximate="tanh")


def linear(x, w, b=None):
    return F.linear(x, w, b)


def timestep_embedding(t, dim, flip_sin_to_cos=False, downscale_freq_shift=1.0, scale=1.0,
                       max_period=10000):
    """difflet/layers/embeddings.py:422-473 (get_timestep_embedding)."""
    half = dim // 2
    exponent = -math.log(max_period) * torch.arange(0, half, dtype=torch.float32)
    exponent = exponent / (half - downscale_freq_shift)
    emb = torch.exp(exponent)
    emb = t[:, None].float() * emb[None, :]
    emb = scale * emb
    emb = torch.cat([torch.sin(emb), torch.cos(emb)], dim=-1)
    if flip_sin_to_cos:
        emb = torch.cat([emb[:, half:], emb[:, :half]], dim=-1)
    if dim % 2 == 1:
        emb = F.pad(emb, (0, 1, 0, 0))
    return emb


def rotary_1d(dim, pos, theta=10000.0):
    """get_1d_rotary_pos_embed(use_real=True, repeat_interleave_real=True, float64 freqs)
    (difflet/layers/embeddings.py:178-244): cos/sin [S, dim] in fp32."""
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64)[: dim // 2] / dim))
    freqs = torch.outer(pos.to(torch.float64), freqs)
    return (freqs.cos().repeat_interleave(2, dim=1).float(),
            freqs.sin().repeat_interleave(2, dim=1).float())


def flux_pos_embed(ids, axes_dim=(16, 56, 56), theta=10000):
    """FluxPosEmbed (difflet/layers/embeddings.py:148-176): per-axis tables concatenated."""
    cos, sin = [], []
    pos = ids.float()
    for i, d in enumerate(axes_dim):
        c, s = rotary_1d(d, pos[:, i], theta)
        cos.append(c)
        sin.append(s)
    return torch.cat(cos, dim=-1), torch.cat(sin, dim=-1)


def flux_ids(txt_len, h, w):
    """FLUX position ids: text tokens (0, 0, 0), image patch (i, j) -> (0, i, j), text first."""
    txt = torch.zeros(txt_len, 3)
    img = torch.zeros(h, w, 3)
    img[..., 1] = torch.arange(h)[:, None]
    img[..., 2] = torch.arange(w)[None, :]
    return torch.cat([txt, img.reshape(h * w, 3)], dim=0)
