"""FLUX on the rocm backend: the fused denoise step as a GPU component and the adapter
FluxPipeline calls (difflet/backends/cuda/flux/)."""

from difflet_amd.backends.rocm.flux.transformer import (TEXT_SEQ_LEN, FluxDiTAdapter,
                                                        RocmFluxTransformerApplication)

__all__ = ["FluxDiTAdapter", "RocmFluxTransformerApplication", "TEXT_SEQ_LEN"]
