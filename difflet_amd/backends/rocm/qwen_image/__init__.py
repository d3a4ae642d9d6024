"""Qwen-Image on the rocm backend: the fused denoise step as a GPU component
(difflet/backends/cuda/qwen_image/)."""

from difflet_amd.backends.rocm.qwen_image.transformer import (
    CHECKPOINT_PREFIX, RocmQwenImageTransformerApplication, transformer_dir)

__all__ = ["CHECKPOINT_PREFIX", "RocmQwenImageTransformerApplication", "transformer_dir"]
