"""The rocm runtime: the platform in difflet_amd.platforms.rocm under the reference's
historical names (difflet/backends/rocm/runtime.py:1-6)."""

from difflet_amd.platforms.rocm import RocmPlatform as RocmBackend
from difflet_amd.platforms.rocm import create_platform as create_backend

__all__ = ["RocmBackend", "create_backend"]
