"""Attention for the rocm backend: the HIP flash-attention kernel (difflet_rocm_attention).

Contract (difflet/ops/attention.py:4-34; the CPU oracle difflet/backends/cpu/ops_impl/
attention.py:8-48; the CUDA twin difflet/backends/cuda/ops_impl/attention.py:41-93):

* ``scale=None`` means 1.0.
* ``attention_mask`` is bool (True = attend) or additive; ``bound_min``/``bound_max`` (both or
  neither, exclusive with a mask) select a per-query key window. Masked scores take the lowest
  finite value, so a fully masked row averages ``v`` as the reference's softmax does.
* ``causal`` masks keys after the query (top-left aligned triangle).
* ``tp_q``/``tp_k``/``tp_out`` are Trainium kernel hints: accepted and ignored.
* Inputs ``(B, H, S, D)`` or ``(B*H, S, D)``, any strides with a contiguous last dim; softmax in
  fp32, output in ``v``'s dtype.

The kernels run bf16 and fp16 on the matrix cores and fp32 on the vector ALUs (an fp32 model
computes in fp32, as the reference's CPU op does), at head_dim 128 (the DiTs) or 64 (the T5 /
UMT5 text encoders). Any other head_dim up to 128 runs on the same kernels with q, k and v
zero-padded to the next of those two: the padded dimensions add exact zeros to every score and
give zero output columns, which are cut off, so the result is the unpadded attention's (the
scale is the caller's, never derived from the padded width). Other dtypes and head_dim above
128 raise NotImplementedError (no silent fallback to another implementation).

The context-parallel forms run their cp = 1 degenerate case (plain attention over the local,
here whole, sequence: difflet/backends/cpu/ops_impl/attention.py:55-143); cp > 1 raises.
"""

from __future__ import annotations

import torch

from difflet_amd.backends.rocm.ops_impl import library

_SUPPORTED = (torch.bfloat16, torch.float16, torch.float32)
_HEAD_DIMS = (64, 128)  # the kernels' own; others up to 128 are zero-padded to one of them


def kernel_head_dim(d: int) -> int:
    """The kernel head_dim that head_dim d runs at: d itself for 64 and 128, else the next of
    the two (d <= 128); NotImplementedError above 128."""
    if d in _HEAD_DIMS:
        return d
    if 0 < d <= 128:
        return 64 if d < 64 else 128
    raise NotImplementedError(f"rocm attention supports head_dim up to 128, got {d}")


def pad_head_dim(t: torch.Tensor, width: int) -> torch.Tensor:
    """t with its last dimension zero-padded to `width` (a new contiguous tensor)."""
    return torch.nn.functional.pad(t, (0, width - t.shape[-1])).contiguous()


def _check(q, k, v):
    for t in (q, k, v):
        if t.device.type != "cuda":
            raise ValueError(f"rocm attention takes device tensors, got one on {t.device}")
    if q.dtype not in _SUPPORTED:
        raise NotImplementedError(
            f"rocm attention runs bf16 / fp16 / fp32 on the HIP kernels; got {q.dtype}")
    if not (q.shape[-1] == k.shape[-1] == v.shape[-1]):
        raise ValueError(f"q, k, v head dims differ: {q.shape[-1]}, {k.shape[-1]}, {v.shape[-1]}")
    kernel_head_dim(q.shape[-1])


def attention(q, k, v, *, scale: float | None = None, causal: bool = False,
              attention_mask=None, bound_min=None, bound_max=None, tp_q: bool = False,
              tp_k: bool = False, tp_out: bool = False, **kwargs):
    del tp_q, tp_k, tp_out, kwargs
    if (bound_min is None) != (bound_max is None):
        raise ValueError("bound_min and bound_max must both be provided")
    if bound_min is not None and attention_mask is not None:
        raise ValueError("attention_mask and bounds are mutually exclusive")
    _check(q, k, v)
    scale = 1.0 if scale is None else float(scale)
    if attention_mask is not None and attention_mask.dtype not in (torch.bool,) + _SUPPORTED:
        attention_mask = attention_mask.to(q.dtype)
    d = q.shape[-1]
    dk = kernel_head_dim(d)
    if dk != d:
        q, k, v = (pad_head_dim(t, dk) for t in (q, k, v))
        out = library.attention(q, k, v, scale, bool(causal), attention_mask, bound_min, bound_max)
        return out[..., :d]
    return library.attention(q, k, v, scale, bool(causal), attention_mask, bound_min, bound_max)


def cross_attention(q, k, v, *, scale: float | None = None, attention_mask=None, **kwargs):
    kwargs.pop("tp_q", None)
    kwargs.pop("tp_k", None)
    kwargs.pop("tp_out", None)
    return attention(q, k, v, scale=scale, causal=False, attention_mask=attention_mask, **kwargs)


def _require_cp1(what: str):
    from difflet_amd.backends.rocm.ops_impl import collectives

    if collectives.get_cp_group().size() != 1:
        raise NotImplementedError(
            f"{what}: context parallelism across GPUs is not implemented on the rocm backend "
            "(this build runs one GPU); run with cp_degree=1")


def ring_attention(q, k, v, *, scale: float, causal: bool = False):
    _require_cp1("ring_attention")
    return attention(q, k, v, scale=scale, causal=causal)


def ulysses_attention(q, k, v, *, scale: float, causal: bool = False):
    _require_cp1("ulysses_attention")
    return attention(q, k, v, scale=scale, causal=causal)


def _valid_prefix_bounds(b, h, s_q, count, device):
    bound_max = count.to(device=device, dtype=torch.int32).reshape(b, 1, 1, 1).expand(b, h, s_q, 1)
    return torch.zeros_like(bound_max), bound_max


def joint_ring_attention(q, image_k, image_v, text_k, text_v, *, scale: float,
                         causal: bool = False, text_valid_len=None):
    """cp = 1: full joint attention over the keys [image | text]; with ``text_valid_len`` the
    keys [0, S_img + count) attend (right-padded text)."""
    _require_cp1("joint_ring_attention")
    k = torch.cat([image_k, text_k], dim=2)
    v = torch.cat([image_v, text_v], dim=2)
    bounds = {}
    if text_valid_len is not None:
        b, h, s_q, _ = q.shape
        count = image_k.shape[2] + text_valid_len.to(torch.int32)
        bounds = dict(zip(("bound_min", "bound_max"), _valid_prefix_bounds(b, h, s_q, count, q.device)))
    return attention(q, k, v, scale=scale, causal=causal, **bounds)


def joint_ulysses_attention(q_img, q_txt, image_k, image_v, text_k, text_v, *, scale: float,
                            causal: bool = False, key_valid_len=None):
    """cp = 1: full joint attention of [q_img | q_txt] over [image | text] keys, split back."""
    _require_cp1("joint_ulysses_attention")
    q = torch.cat([q_img, q_txt], dim=2)
    k = torch.cat([image_k, text_k], dim=2)
    v = torch.cat([image_v, text_v], dim=2)
    bounds = {}
    if key_valid_len is not None:
        b, h, s_q, _ = q.shape
        bounds = dict(zip(("bound_min", "bound_max"),
                          _valid_prefix_bounds(b, h, s_q, key_valid_len, q.device)))
    out = attention(q, k, v, scale=scale, causal=causal, **bounds)
    s_img = q_img.shape[2]
    return out[:, :, :s_img], out[:, :, s_img:]


__all__ = [
    "attention",
    "cross_attention",
    "joint_ring_attention",
    "joint_ulysses_attention",
    "ring_attention",
    "ulysses_attention",
]
