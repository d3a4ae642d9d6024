"""The rocm backend: Difflet's `difflet.ops` surface on the gfx950 HIP kernels.

Mirrors difflet/backends/rocm/__init__.py (the reference's placeholder): `RocmBackend` /
`create_backend` under their historical names, and `ops_impl/` with the eight modules
difflet/ops/_dispatch.py:10-20 imports by name (attention, collectives, embeddings, linear,
markers, mx, norm, platform).
"""

from difflet_amd.backends.rocm.runtime import RocmBackend, create_backend

__all__ = ["RocmBackend", "create_backend"]
