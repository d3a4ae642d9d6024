"""Linear / embedding layers for the rocm backend at tp = 1, on the HIP GEMM / GEMV.

Same constructors, attributes, state dicts and bias semantics as the CPU twins
(difflet/backends/cpu/ops_impl/linear.py:9-54) and the shared torch layers
(difflet/backends/_torch_megatron/linear.py:88-210): ``skip_bias_add`` returns
``(x @ W^T, bias)``; ``reduce_output`` / ``gather_output`` / ``input_is_parallel`` /
``reduce_dtype`` are accepted and have no effect at tp = 1.

The matmul: bf16 weights run the bf16 kernels, up to 8 rows of input through the GEMV kernel
(the modulation and timestep linears, HBM-bound on W), more through the tiled GEMM; fp32
weights (a model loaded in fp32, such as the T5 encoders' fp32 option) run the fp32
matrix-core GEMM, in fp32 throughout as F.linear does. A K or N off the kernel's multiples (64
and 4 for bf16, 4 and 4 for fp32) is zero-padded once on the weight (and per call on the input).
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from difflet_amd.backends.rocm.ops_impl import library


class _RocmLinearBase(nn.Module):
    def _init_linear(self, in_features: int, out_features: int, bias: bool, dtype=None,
                     device=None):
        self.in_features, self.out_features = int(in_features), int(out_features)
        self.input_size, self.output_size = self.in_features, self.out_features
        factory = {"dtype": dtype, "device": device}
        self.weight = nn.Parameter(torch.empty(out_features, in_features, **factory))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, **factory))
        else:
            self.register_parameter("bias", None)
        self._padded = None
        self.reset_parameters()

    def reset_parameters(self):
        if self.weight.device.type == "meta":
            return
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            bound = 1 / math.sqrt(self.in_features) if self.in_features > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

    def _weight_for_gemm(self):
        w = self.weight
        k, n = self.in_features, self.out_features
        kq = 64 if w.dtype == torch.bfloat16 else 4
        kp, np_ = -(-k // kq) * kq, -(-n // 4) * 4
        if kp == k and np_ == n:
            return w.detach(), k, n
        key = (w.data_ptr(), w._version)
        if self._padded is None or self._padded[0] != key:
            wp = torch.zeros(np_, kp, dtype=w.dtype, device=w.device)
            wp[:n, :k] = w.detach()
            self._padded = (key, wp)
        return self._padded[1], kp, np_

    def _matmul(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        w = self.weight
        if x.device.type != "cuda" or w.device.type != "cuda":
            raise ValueError("rocm linear takes device tensors")
        if w.dtype == torch.float32:
            return self._matmul_f32(x, bias)
        if w.dtype != torch.bfloat16:
            raise NotImplementedError(f"rocm linear runs bf16 or fp32 weights, got {w.dtype}")
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.dtype != torch.bfloat16:
            x2 = x2.to(torch.bfloat16)
        b = None if bias is None else bias.detach().to(torch.bfloat16)
        m = x2.shape[0]
        if m == 0:
            return x.new_empty(*shape[:-1], self.out_features)
        # a few rows run on the GEMV kernel with the weight as is; the GEMM reads the weight
        # zero-padded to its tile multiples (built once, only for odd shapes)
        wg = w.detach() if library._gemv_fits(m, self.in_features) else self._weight_for_gemm()[0]
        y = library.linear(x2, wg, b, self.out_features)
        return y.reshape(*shape[:-1], self.out_features).to(x.dtype)


    def _matmul_f32(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).to(torch.float32)
        m = x2.shape[0]
        if m == 0:
            return x.new_empty(*shape[:-1], self.out_features)
        b = None if bias is None else bias.detach().to(torch.float32)
        y = library.linear_f32(x2, self._weight_for_gemm()[0], b, self.out_features)
        return y.reshape(*shape[:-1], self.out_features).to(x.dtype)


class ColumnParallelLinear(_RocmLinearBase):
    def __init__(self, input_size, output_size, bias=True, gather_output=True, dtype=None,
                 device=None, **kwargs):
        super().__init__()
        del kwargs
        self.gather_output = gather_output
        self._init_linear(input_size, output_size, bias, dtype, device)

    def forward(self, x):
        return self._matmul(x, self.bias)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, bias={self.bias is not None}"


class RowParallelLinear(_RocmLinearBase):
    def __init__(self, input_size, output_size, bias=True, input_is_parallel=False,
                 reduce_output=True, skip_bias_add=False, dtype=None, device=None, **kwargs):
        super().__init__()
        del kwargs
        self.input_is_parallel = input_is_parallel
        self.reduce_output = reduce_output
        self.skip_bias_add = skip_bias_add
        self.tensor_parallel_group = None
        self._init_linear(input_size, output_size, bias, dtype, device)

    def forward(self, x):
        if self.skip_bias_add:
            return self._matmul(x, None), self.bias
        return self._matmul(x, self.bias)

    def extra_repr(self) -> str:
        return (f"in={self.in_features}, out={self.out_features}, bias={self.bias is not None}, "
                f"skip_bias_add={self.skip_bias_add}")


class ParallelEmbedding(nn.Embedding):
    """nn.Embedding at tp = 1 (a gather, not on the denoise step's path)."""

    def __init__(self, num_embeddings, embedding_dim, shard_across_embedding=False, pad=False,
                 **kwargs):
        del shard_across_embedding, pad, kwargs
        super().__init__(num_embeddings, embedding_dim)


__all__ = ["ColumnParallelLinear", "ParallelEmbedding", "RowParallelLinear"]
