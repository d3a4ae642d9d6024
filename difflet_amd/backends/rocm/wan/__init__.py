"""Wan on the rocm backend: one DiT expert's fused denoise step as a GPU component
(difflet/backends/cuda/wan/)."""

from difflet_amd.backends.rocm.wan.transformer import RocmWanTransformerApplication

__all__ = ["RocmWanTransformerApplication"]
