"""The ROCm platform: the generic GPU flow on MI355X (gfx950) with the rocm backend's ops.

Replaces the reserved placeholder difflet/platforms/rocm.py:8-23 (whose prepare_runtime
raises). Inside a Difflet tree it subclasses difflet.platforms.gpu.GpuPlatform, so the GPU flow
(device type "cuda" under PyTorch-ROCm, difflet/platforms/gpu.py:23-97) runs unchanged; on its
own it carries the same attributes.

One GPU per process, one process: a launch with WORLD_SIZE > 1 is refused (the build does not
implement collectives across GPUs).
"""

from __future__ import annotations

import hashlib
import os

try:  # inside a Difflet tree
    from difflet.platforms.gpu import GpuPlatform as _Base
except ImportError:  # standalone
    class _Base:  # noqa: D401 - the attributes the GPU flow reads
        device_type = "cuda"
        distributed_backend = "nccl"

        def device_available(self) -> bool:
            import torch

            return bool(torch.cuda.is_available())

        def set_current_device(self, index: int) -> None:
            import torch

            torch.cuda.set_device(index)


class RocmPlatform(_Base):
    name = "rocm"
    display_name = "ROCm"
    visible_devices_var = "HIP_VISIBLE_DEVICES"
    gfx_arch = "gfx950"

    @classmethod
    def detect(cls) -> bool:
        """PyTorch-ROCm with a gfx950 device visible. (Difflet tries CUDA first and
        CudaPlatform.detect only asks torch.cuda.is_available(), which is true on ROCm too:
        select DIFFLET_BACKEND=rocm, or have CUDA detection check torch.version.hip.)"""
        import torch

        if not getattr(torch.version, "hip", None) or not torch.cuda.is_available():
            return False
        try:
            return any(cls.gfx_arch in torch.cuda.get_device_properties(i).gcnArchName
                       for i in range(torch.cuda.device_count()))
        except Exception:
            return False

    def prepare_runtime(self, parallel=None) -> None:
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("DIFFLET_BACKEND=rocm selected but no ROCm device is visible")
        world = int(os.environ.get("WORLD_SIZE", "1"))
        if world > 1:
            raise NotImplementedError(
                f"WORLD_SIZE={world}: the rocm backend runs one GPU per process and no "
                "collectives across GPUs in this build")
        self.set_current_device(int(os.environ.get("LOCAL_RANK", "0")))
        from difflet_amd import _lib

        _lib.load()  # the kernels must be there; no silent fallback

    def toolchain_versions(self) -> dict:
        import torch

        from difflet_amd import _lib

        out = {"torch": torch.__version__, "hip": getattr(torch.version, "hip", None)}
        if _lib.LIB_PATH.exists():
            out["difflet_rocm"] = _lib.load().difflet_rocm_version().decode()
            out["difflet_rocm_sha256"] = hashlib.sha256(_lib.LIB_PATH.read_bytes()).hexdigest()[:16]
        return out


def create_platform() -> RocmPlatform:
    return RocmPlatform()
