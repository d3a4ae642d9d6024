"""Normalization layers for the rocm backend on the HIP kernels.

LayerNorm      -- the nn.LayerNorm signature and state dict (``weight``, ``bias``), normalizing
                  the last dimension (difflet/backends/cpu/ops_impl/norm.py:9); fp32 statistics.
RMSNorm        -- (hidden_size, eps=1e-6) with one ``weight`` (the state dict of
                  difflet/backends/cpu/ops_impl/norm.py:12-22); computed with the fp32 law of
                  the CUDA backend (difflet/backends/cuda/ops_impl/norm.py:28-44): fp32
                  statistics, normalisation and affine, one cast back. The CPU module
                  normalises in the input dtype; the two agree within bf16 rounding.
rms_norm_fp32  -- difflet/backends/_torch_megatron/norm.py:35-45 on the kernel.
"""

from __future__ import annotations

import numbers

import torch
import torch.nn as nn

from difflet_amd.backends.rocm.ops_impl import library


def rms_norm_fp32(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    if x.shape[-1] % 8:
        raise NotImplementedError(f"rocm rms_norm needs the last dim a multiple of 8, got {x.shape[-1]}")
    return library.rms_norm(x, weight, float(eps))


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6, **kwargs):
        super().__init__()
        del kwargs
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return rms_norm_fp32(hidden_states, self.weight, self.eps)


CustomRMSNorm = RMSNorm


class LayerNorm(nn.Module):
    def __init__(self, normalized_shape, eps: float = 1e-5, elementwise_affine: bool = True,
                 bias: bool = True, device=None, dtype=None):
        super().__init__()
        if isinstance(normalized_shape, numbers.Integral):
            normalized_shape = (int(normalized_shape),)
        self.normalized_shape = tuple(normalized_shape)
        if len(self.normalized_shape) != 1:
            raise NotImplementedError("rocm LayerNorm normalizes the last dimension only")
        self.eps = eps
        self.elementwise_affine = elementwise_affine
        factory = {"device": device, "dtype": dtype}
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(self.normalized_shape, **factory))
            self.bias = nn.Parameter(torch.zeros(self.normalized_shape, **factory)) if bias else None
        else:
            self.register_parameter("weight", None)
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.normalized_shape[0]:
            raise ValueError(f"LayerNorm over {self.normalized_shape}, got input {tuple(x.shape)}")
        if x.shape[-1] % 8:
            raise NotImplementedError("rocm LayerNorm needs the last dim a multiple of 8")
        return library.layer_norm(x, self.weight, self.bias, float(self.eps))

    def extra_repr(self) -> str:
        return f"{self.normalized_shape}, eps={self.eps}, elementwise_affine={self.elementwise_affine}"


__all__ = ["CustomRMSNorm", "LayerNorm", "RMSNorm", "rms_norm_fp32"]
