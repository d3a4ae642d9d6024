"""The quantized-linear API on the rocm backend: spec (RocmQuantSpec, target sets) and the fp8
twin layers (quantize_module_, prepare_fp8_kernels_, FusedFP8Projections)."""
