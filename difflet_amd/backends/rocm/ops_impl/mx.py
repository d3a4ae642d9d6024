"""The op surface's MX ops (the Trainium 8 x 4 packed law of difflet/backends/cpu/ops_impl/mx.py)
on the rocm backend: deliberately unimplemented, as on CUDA
(difflet/backends/cuda/ops_impl/mx.py:9-25). No GPU model calls them; silently running another
precision than the one asked for would be worse than refusing. The MXFP8 linear law of
difflet/quant/mx.py, which the GPU models do use, is implemented in difflet_amd.quant."""

_UNSUPPORTED = ("the op surface's Trainium MX ops are not implemented on the rocm backend; "
                "MXFP8 linears go through difflet_amd.quant (quantize_module_)")


def quantize_mx(*args, **kwargs):
    raise NotImplementedError(f"quantize_mx: {_UNSUPPORTED}")


def dequantize_mx(*args, **kwargs):
    raise NotImplementedError(f"dequantize_mx: {_UNSUPPORTED}")


def linear_mx(*args, **kwargs):
    raise NotImplementedError(f"linear_mx: {_UNSUPPORTED}")


def matmul_mx(*args, **kwargs):
    raise NotImplementedError(f"matmul_mx: {_UNSUPPORTED}")


__all__ = ["dequantize_mx", "linear_mx", "matmul_mx", "quantize_mx"]
