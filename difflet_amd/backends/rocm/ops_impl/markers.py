"""Layer-boundary markers: a no-op on this backend, as on CPU
(difflet/backends/cpu/ops_impl/markers.py:11-20). One tensor in returns that tensor; several
return the tuple. The Trainium compiler is the only consumer of the markers."""

from torch import nn


class _Passthrough(nn.Module):
    def forward(self, *tensors):
        return tensors[0] if len(tensors) == 1 else tensors


class ModuleMarkerStartWrapper(_Passthrough):
    pass


class ModuleMarkerEndWrapper(_Passthrough):
    pass


__all__ = ["ModuleMarkerEndWrapper", "ModuleMarkerStartWrapper"]
