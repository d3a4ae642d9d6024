"""fp8 linears for the rocm backend: the device side of the quantized-linear API.

The rocm twins of the neuron backend's FP8 layers (difflet/backends/neuron/ops_impl/
fp8_linear.py:60-432): the same constructor arguments and bias semantics as the backend's
ColumnParallelLinear / RowParallelLinear / nn.Linear, the weight stored as ``float8_e4m3fn`` as
the quantized checkpoint holds it, beside its scales:

* ``mxfp8``       -- ``weight_scale`` uint8 E8M0 ``[out, in/32]`` in the reference's block law
                     (difflet/quant/mx.py); codes in logical K order;
* ``fp8_rowwise`` -- ``weight_scale`` fp32 ``[out]``, one per output channel.

``compute="rocm"``: after the load, prepare_kernel_() lays the weight out for the HIP GEMM (MX
codes permuted to swizzle order, so the GEMM's contiguous 32-K blocks are the law's blocks);
each call quantizes the bf16 activation on the device (per token, or per MX block in the same
order) and runs the fp8 GEMM with fp32 accumulation, bf16 out. ``compute="dequant"``: the weight
is dequantized once to bf16 and the bf16 GEMM runs (memory only). Inference only.
"""

from __future__ import annotations

from collections.abc import Callable

import torch
import torch.nn as nn

from difflet_amd import kernels
from difflet_amd.backends.rocm.ops_impl import library
from difflet_amd.quant.spec import BLOCK, LAYOUT_K, RocmQuantSpec

FP8_DTYPE = torch.float8_e4m3fn


def _swizzle_index(k: int, device) -> torch.Tensor:
    """perm[r * 4 + j] = k0 + j * (tile / 4) + r over 512-wide tiles and a remainder tile
    (difflet/quant/mx.py:46-76), as a gather index on the device."""
    parts, k0 = [], 0
    while k0 < k:
        t = 512 if k - k0 >= 512 else k - k0
        parts.append(torch.arange(k0, k0 + t).reshape(4, t // 4).t().reshape(-1))
        k0 += t
    return torch.cat(parts).to(device)


def _e4m3_values(dev):
    return torch.arange(256, dtype=torch.uint8, device=dev).view(FP8_DTYPE).to(torch.float32)


class _FP8LinearBase(nn.Module):
    def _init_tensors(self, out_f: int, in_f: int, bias: bool, *, dtype, device, compute: str,
                      fmt: str) -> None:
        if compute not in ("rocm", "dequant"):
            raise ValueError(f"fp8 compute must be 'rocm' or 'dequant', got {compute!r}")
        if fmt == "mxfp8" and in_f % LAYOUT_K:
            raise ValueError(f"mxfp8 needs in_features a multiple of {LAYOUT_K}, got {in_f}")
        if fmt == "fp8_rowwise" and in_f % 128:
            raise ValueError(f"the fp8 GEMM needs in_features a multiple of 128, got {in_f}")
        self.compute, self.format = compute, fmt
        self.in_features, self.out_features = int(in_f), int(out_f)
        self.input_size, self.output_size = self.in_features, self.out_features
        self.weight = nn.Parameter(torch.empty(out_f, in_f, dtype=FP8_DTYPE, device=device),
                                   requires_grad=False)
        if fmt == "mxfp8":
            self.register_buffer("weight_scale", torch.zeros(out_f, in_f // BLOCK,
                                                             dtype=torch.uint8, device=device))
        else:
            self.register_buffer("weight_scale", torch.ones(out_f, dtype=torch.float32,
                                                            device=device))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_f, dtype=dtype or torch.bfloat16,
                                                 device=device), requires_grad=False)
        else:
            self.register_parameter("bias", None)
        self.register_buffer("weight_kernel", None, persistent=False)
        self.register_buffer("weight_bf16", None, persistent=False)

    # ---------------------------------------------------------------- weights
    @torch.no_grad()
    def load_from_dense_(self, weight: torch.Tensor, bias: torch.Tensor | None = None) -> None:
        """Quantize a dense (bf16 / fp32) weight into this layer on the device, by the layer's
        format: what the quantized checkpoint writer would store."""
        w = weight.to(device=self.weight.device, dtype=torch.bfloat16).contiguous()
        if self.format == "mxfp8":
            q, s = kernels.quantize_mxfp8(w, swizzled=False)
        else:
            q, s = kernels.quantize_fp8_rowwise(w)
        self.weight.data = q
        self.weight_scale = s
        if bias is not None and self.bias is not None:
            self.bias.data = bias.to(device=self.weight.device, dtype=self.bias.dtype)
        self.weight_kernel = None
        self.weight_bf16 = None

    @torch.no_grad()
    def dequantized(self) -> torch.Tensor:
        """fp32 [out, in] of the stored codes and scales."""
        w = self.weight if self.weight is not None else None
        if w is None:
            raise RuntimeError("the fp8 weight was dropped by prepare_kernel_")
        vals = _e4m3_values(w.device)[w.view(torch.uint8).long()]
        if self.format == "mxfp8":
            scale = torch.exp2(self.weight_scale.float() - 127.0)
            return (vals.view(self.out_features, -1, BLOCK) * scale[..., None]).reshape(vals.shape)
        return vals * self.weight_scale[:, None]

    @torch.no_grad()
    def prepare_kernel_(self) -> None:
        """After the load: the kernel's layout (rocm) or the bf16 weight (dequant); the logical
        fp8 weight is then dropped. A no-op once done."""
        if self.weight is None:
            return
        if self.compute == "dequant":
            self.weight_bf16 = self.dequantized().to(torch.bfloat16)
        elif self.format == "mxfp8":
            idx = _swizzle_index(self.in_features, self.weight.device)
            self.weight_kernel = self.weight.data.view(torch.uint8)[:, idx].contiguous()
        else:
            self.weight_kernel = self.weight.data.view(torch.uint8).contiguous()
        self.weight = None

    # ---------------------------------------------------------------- matmul
    def _matmul(self, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.dtype != torch.bfloat16:
            x2 = x2.to(torch.bfloat16)
        b = None if bias is None else bias.detach().to(torch.bfloat16)
        if self.compute == "dequant":
            if self.weight_bf16 is None:
                raise RuntimeError("call prepare_fp8_kernels_(module) after the load")
            y = library.linear(x2, self.weight_bf16, b, self.out_features)
        else:
            if self.weight_kernel is None:
                raise RuntimeError("the fp8 kernel path needs the prepared weight: call "
                                   "prepare_fp8_kernels_(module) after the load")
            y = library.fp8_linear(x2, self.weight_kernel, self.weight_scale, b,
                                   self.format == "mxfp8")
        return y.reshape(*shape[:-1], self.out_features).to(x.dtype)

    def _repr_tail(self) -> str:
        return f"compute={self.compute}, {self.format}"


class FP8Linear(_FP8LinearBase):
    def __init__(self, in_features, out_features, bias=True, *, dtype=None, device=None,
                 compute="rocm", format="mxfp8"):
        super().__init__()
        self._init_tensors(out_features, in_features, bias, dtype=dtype, device=device,
                           compute=compute, fmt=format)

    def forward(self, x):
        return self._matmul(x, self.bias)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, {self._repr_tail()}"


class FP8ColumnParallelLinear(FP8Linear):
    def __init__(self, input_size, output_size, bias=True, gather_output=True, dtype=None,
                 device=None, compute="rocm", format="mxfp8", **kwargs):
        del kwargs
        super().__init__(input_size, output_size, bias, dtype=dtype, device=device,
                         compute=compute, format=format)
        self.gather_output = gather_output


class FP8RowParallelLinear(_FP8LinearBase):
    def __init__(self, input_size, output_size, bias=True, input_is_parallel=False, dtype=None,
                 device=None, reduce_output=True, skip_bias_add=False, compute="rocm",
                 format="mxfp8", **kwargs):
        super().__init__()
        del kwargs
        self.input_is_parallel, self.reduce_output = input_is_parallel, reduce_output
        self.skip_bias_add = skip_bias_add
        self.tensor_parallel_group = None
        self._init_tensors(output_size, input_size, bias, dtype=dtype, device=device,
                           compute=compute, fmt=format)

    def forward(self, x):
        if self.skip_bias_add:
            return self._matmul(x, None), self.bias
        return self._matmul(x, self.bias)

    def extra_repr(self) -> str:
        return (f"in={self.in_features}, out={self.out_features}, "
                f"skip_bias_add={self.skip_bias_add}, {self._repr_tail()}")


def _parallel_kind(linear: nn.Module) -> str | None:
    """difflet/backends/neuron/ops_impl/fp8_linear.py:243-258: by class name, since model code
    binds whichever backend's ColumnParallelLinear was selected when it was imported."""
    name = type(linear).__name__
    if name == "ColumnParallelLinear":
        return "column"
    if name == "RowParallelLinear":
        return "row"
    return None


def fp8_twin(linear: nn.Module, *, compute: str, format: str) -> _FP8LinearBase:
    weight = linear.weight
    factory = {"dtype": weight.dtype if weight.dtype != FP8_DTYPE else torch.bfloat16,
               "device": weight.device, "compute": compute, "format": format}
    has_bias = getattr(linear, "bias", None) is not None
    n_in = getattr(linear, "input_size", getattr(linear, "in_features", None))
    n_out = getattr(linear, "output_size", getattr(linear, "out_features", None))
    kind = _parallel_kind(linear)
    if kind == "column":
        return FP8ColumnParallelLinear(n_in, n_out, bias=has_bias,
                                       gather_output=getattr(linear, "gather_output", True),
                                       **factory)
    if kind == "row":
        return FP8RowParallelLinear(n_in, n_out, bias=has_bias,
                                    input_is_parallel=getattr(linear, "input_is_parallel", False),
                                    reduce_output=getattr(linear, "reduce_output", True),
                                    skip_bias_add=getattr(linear, "skip_bias_add", False),
                                    **factory)
    if isinstance(linear, nn.Linear):
        return FP8Linear(n_in, n_out, bias=has_bias, **factory)
    raise TypeError(f"cannot quantize a {type(linear).__name__}")


def _is_linear(m: nn.Module) -> bool:
    return (isinstance(m, nn.Linear) or _parallel_kind(m) is not None) and not isinstance(
        m, _FP8LinearBase)


def quantize_module_(module: nn.Module, spec: RocmQuantSpec, *,
                     key_fn: Callable[[str], str] | None = None,
                     from_dense: bool = False) -> list[str]:
    """difflet/backends/neuron/ops_impl/fp8_linear.py:288-335: replace every linear the spec
    targets with its fp8 twin, in place; returns the replaced names. A target pattern that
    matches no linear is refused. ``from_dense=True`` quantizes each replaced layer's current
    dense weight into its twin on the device (synthetic or unquantized checkpoints); otherwise
    the twins are empty, for the quantized checkpoint's loader to fill."""
    key = ((lambda name: key_fn(f"{name}.weight").removesuffix(".weight"))
           if key_fn is not None else (lambda name: name))
    linears = [(n, c) for n, c in module.named_modules() if _is_linear(c)]
    dead = spec.unmatched_targets(key(n) for n, _ in linears)
    if dead:
        raise ValueError(f"quantization target patterns match no linear in the module: {dead}")
    targets = [(n, c) for n, c in linears if spec.matches(key(n))]
    twins = []
    for name, child in targets:
        try:
            twin = fp8_twin(child, compute=spec.compute, format=spec.format)
        except ValueError as exc:
            raise ValueError(f"{name}: {exc}") from exc
        if from_dense:
            twin.load_from_dense_(child.weight.detach(), getattr(child, "bias", None))
        twins.append((name, twin))
    for name, twin in twins:
        parent_path, _, leaf = name.rpartition(".")
        parent = module.get_submodule(parent_path) if parent_path else module
        if isinstance(parent, (nn.ModuleList, nn.Sequential)):
            parent[int(leaf)] = twin
        else:
            setattr(parent, leaf, twin)
    return [n for n, _ in targets]


def fp8_linears(module: nn.Module) -> list[str]:
    return [n for n, c in module.named_modules() if isinstance(c, _FP8LinearBase)]


class FusedFP8Projections(nn.Module):
    """Several fp8 projections of one input (q, k, v) as one GEMM: the activation is quantized
    once and the weights are concatenated along N (difflet/backends/neuron/ops_impl/
    fp8_linear.py:343-385). Built from prepared-or-loaded layers of one format."""

    def __init__(self, layers: list[_FP8LinearBase]) -> None:
        super().__init__()
        if not layers or any(l.compute != "rocm" for l in layers):
            raise ValueError("fused projections need fp8 layers on the kernel path")
        if len({l.format for l in layers}) != 1:
            raise ValueError("fused projections must share one format")
        if any(l.weight is None for l in layers):
            raise ValueError("fuse before the layers drop their weights (prepare_kernel_)")
        if len({l.in_features for l in layers}) != 1:
            raise ValueError("fused projections must share the input size")
        biases = [l.bias for l in layers]
        if any(b is None for b in biases) and not all(b is None for b in biases):
            raise ValueError("fused projections must all have a bias or none")
        self.format = layers[0].format
        self.splits = [l.out_features for l in layers]
        fused = FP8Linear(layers[0].in_features, sum(self.splits), bias=biases[0] is not None,
                          device=layers[0].weight.device, compute="rocm", format=self.format)
        with torch.no_grad():
            fused.weight.data = torch.cat([l.weight.data for l in layers], dim=0)
            fused.weight_scale = torch.cat([l.weight_scale for l in layers], dim=0)
            if biases[0] is not None:
                fused.bias.data = torch.cat([b.data.to(torch.bfloat16) for b in biases], dim=0)
        fused.prepare_kernel_()
        self.fused = fused

    def forward(self, x):
        return tuple(self.fused(x).split(self.splits, dim=-1))

    def extra_repr(self) -> str:
        return f"splits={self.splits}, {self.format} rocm"


FUSED_PROJECTION_GROUPS: tuple[tuple[str, tuple[str, ...]], ...] = (
    ("fused_qkv", ("to_q", "to_k", "to_v")),
    ("fused_add_qkv", ("add_q_proj", "add_k_proj", "add_v_proj")),
)


def fuse_projections_(module: nn.Module) -> list[str]:
    fused = []
    for name, child in list(module.named_modules()):
        for attr, members in FUSED_PROJECTION_GROUPS:
            layers = [getattr(child, m, None) for m in members]
            if not all(isinstance(l, _FP8LinearBase) and l.compute == "rocm"
                       and l.weight is not None for l in layers):
                continue
            if any(getattr(l, "gather_output", False) for l in layers):
                continue
            child.add_module(attr, FusedFP8Projections(layers))
            fused.append(f"{name}.{attr}" if name else attr)
    return fused


def prepare_fp8_kernels_(module: nn.Module, *, fuse: bool = False) -> int:
    """difflet/backends/neuron/ops_impl/fp8_linear.py:419-432: prepare every fp8 linear (after
    the load, before the first forward); returns how many were prepared."""
    if fuse:
        fuse_projections_(module)
    count = 0
    for child in module.modules():
        if isinstance(child, _FP8LinearBase):
            child.prepare_kernel_()  # a no-op for a layer already prepared (or fused)
            count += 1
    return count


__all__ = [
    "FP8ColumnParallelLinear", "FP8Linear", "FP8RowParallelLinear", "FUSED_PROJECTION_GROUPS",
    "FusedFP8Projections", "fp8_linears", "fp8_twin", "fuse_projections_",
    "prepare_fp8_kernels_", "quantize_module_",
]
