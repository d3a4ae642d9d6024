"""Platform facts for the rocm backend (difflet/backends/cuda/ops_impl/platform.py:13-22 is the
template). The enum keeps TRN1, which FLUX's modeling compares against
(difflet/models/flux/modeling_flux.py:73,1372,1415)."""

from __future__ import annotations

from enum import Enum


class hardware(Enum):
    CPU = "cpu"
    TRN1 = "trn1"
    TRN2 = "trn2"
    TPU = "tpu"
    CUDA = "cuda"
    ROCM = "rocm"


def get_platform_target():
    return hardware.ROCM


__all__ = ["get_platform_target", "hardware"]
