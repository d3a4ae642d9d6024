"""The rocm kernels as torch custom operators (namespace ``difflet_rocm``).

The op modules call the HIP kernels through these operators, not through ctypes directly: to
``torch.compile`` each one is a single opaque node with a fake (meta) implementation that gives
the output's shape and dtype, so Dynamo traces a block that uses them without a graph break and
Inductor compiles the torch code around them. This is what the reference's CUDA and TPU backends
do for their own fused kernels (difflet/backends/cuda/hunyuan_video_15/modeling.py:73-100,
difflet/backends/tpu/ops_impl/collectives.py:99-150).

Every operator is functional: it allocates and returns a new contiguous tensor and mutates no
argument. Shape and dtype checks that raise for unsupported inputs stay in the op modules, so
they also run while tracing.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from difflet_amd import kernels

Tensor = torch.Tensor


# ---------------------------------------------------------------------------------- attention
@torch.library.custom_op("difflet_rocm::attention", mutates_args=())
def attention(q: Tensor, k: Tensor, v: Tensor, scale: float, causal: bool,
              attention_mask: Optional[Tensor], bound_min: Optional[Tensor],
              bound_max: Optional[Tensor]) -> Tensor:
    """difflet_rocm_attention: (B, H, S, D) or (B*H, S, D) q/k/v, output in v's dtype."""
    return kernels.attention(q, k, v, scale=scale, causal=causal, attention_mask=attention_mask,
                             bound_min=bound_min, bound_max=bound_max).contiguous()


@attention.register_fake
def _(q, k, v, scale, causal, attention_mask, bound_min, bound_max):
    return q.new_empty((*q.shape[:-1], v.shape[-1]), dtype=v.dtype)


# ------------------------------------------------------------------------------------- linear
#: up to this many input rows a linear runs on the GEMV kernel (HBM-bound on the weight)
GEMV_ROWS = 8


def _gemv_fits(m: int, k: int) -> bool:
    """The GEMV kernel stages m rows of x in LDS: m (rounded up to 1, 2, 4 or 8) x k <= 16384."""
    return m <= GEMV_ROWS and k % 8 == 0 and {1: 1, 2: 2}.get(m, 4 if m <= 4 else 8) * k <= 16384


@torch.library.custom_op("difflet_rocm::linear", mutates_args=())
def linear(x: Tensor, w: Tensor, bias: Optional[Tensor], out_features: int) -> Tensor:
    """y [M, out_features] bf16 = x [M, K'] @ w[:out_features, :K']^T + bias, where w [N', K'] may be
    the zero-padded weight (K' a multiple of 64, N' of 4); x is padded to K' here."""
    m, kx = x.shape
    n_pad, k_pad = w.shape
    if m == 0:
        return x.new_empty((0, out_features), dtype=torch.bfloat16)
    if n_pad == out_features and k_pad == kx and _gemv_fits(m, kx):
        return kernels.gemv(x, w, bias)
    if kx != k_pad:
        x = F.pad(x, (0, k_pad - kx))
    if bias is not None and bias.shape[0] != n_pad:
        bias = F.pad(bias, (0, n_pad - bias.shape[0]))
    y = kernels.linear(x if x.stride(-1) == 1 else x.contiguous(), w, bias)
    return y if n_pad == out_features else y[:, :out_features].contiguous()


@linear.register_fake
def _(x, w, bias, out_features):
    return x.new_empty((x.shape[0], out_features), dtype=torch.bfloat16)


@torch.library.custom_op("difflet_rocm::linear_f32", mutates_args=())
def linear_f32(x: Tensor, w: Tensor, bias: Optional[Tensor], out_features: int) -> Tensor:
    """y [M, out_features] fp32 = x [M, K'] @ w[:out_features, :K']^T + bias on the fp32 GEMM,
    where w [N', K'] may be the zero-padded weight (K' and N' multiples of 4)."""
    m, kx = x.shape
    n_pad, k_pad = w.shape
    if m == 0:
        return x.new_empty((0, out_features), dtype=torch.float32)
    if kx != k_pad:
        x = F.pad(x, (0, k_pad - kx))
    if bias is not None and bias.shape[0] != n_pad:
        bias = F.pad(bias, (0, n_pad - bias.shape[0]))
    y = kernels.gemm_f32(x.contiguous(), w, None if bias is None else bias.contiguous())
    return y if n_pad == out_features else y[:, :out_features].contiguous()


@linear_f32.register_fake
def _(x, w, bias, out_features):
    return x.new_empty((x.shape[0], out_features), dtype=torch.float32)


@torch.library.custom_op("difflet_rocm::fp8_linear", mutates_args=())
def fp8_linear(x: Tensor, w_kernel: Tensor, w_scale: Tensor, bias: Optional[Tensor],
               mx: bool) -> Tensor:
    """The fp8 twins' matmul: x [M, K] bf16 quantized per token (per-channel weights) or per MX
    block in swizzle order (mx), then the fp8 GEMM with fp32 accumulation, bf16 [M, N] out."""
    y = torch.empty((x.shape[0], w_kernel.shape[0]), dtype=torch.bfloat16, device=x.device)
    if mx:
        aq, asc = kernels.quantize_mxfp8(x, swizzled=True)
    else:
        aq, asc = kernels.quantize_fp8_rowwise(x)
    kernels.gemm_grouped([kernels.Problem(aq, w_kernel, y, bias, a_scale=asc, w_scale=w_scale)],
                         kind="mx" if mx else "fp8")
    return y


@fp8_linear.register_fake
def _(x, w_kernel, w_scale, bias, mx):
    return x.new_empty((x.shape[0], w_kernel.shape[0]), dtype=torch.bfloat16)


# ---------------------------------------------------------------------------- norms, rotary
@torch.library.custom_op("difflet_rocm::rms_norm", mutates_args=())
def rms_norm(x: Tensor, weight: Optional[Tensor], eps: float) -> Tensor:
    """difflet_rocm_rms_norm: the fp32 RMSNorm law, one cast back to x's dtype."""
    return kernels.rms_norm(x, weight, eps)


@rms_norm.register_fake
def _(x, weight, eps):
    return x.new_empty(x.shape)


@torch.library.custom_op("difflet_rocm::layer_norm", mutates_args=())
def layer_norm(x: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], eps: float) -> Tensor:
    """difflet_rocm_layernorm_modulate with one_plus = 0: LN(x) * weight + bias, fp32 stats."""
    return kernels.layernorm_modulate(x, weight, bias, eps=eps, one_plus=False)


@layer_norm.register_fake
def _(x, weight, bias, eps):
    return x.new_empty(x.shape)


@torch.library.custom_op("difflet_rocm::rope", mutates_args=())
def rope(x: Tensor, cos: Tensor, sin: Tensor, law: int) -> Tensor:
    """difflet_rocm_rope on x [..., S, D] with fp32 tables [S, D]; law 0 rotates in fp32
    (apply_rotary_emb_fp32), law 1 in the input dtype (apply_rotary_emb)."""
    return kernels.rope(x, cos, sin, law=law)


@rope.register_fake
def _(x, cos, sin, law):
    return x.new_empty(x.shape)


__all__ = ["attention", "fp8_linear", "layer_norm", "linear", "rms_norm", "rope"]
