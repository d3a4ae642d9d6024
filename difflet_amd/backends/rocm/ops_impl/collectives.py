"""Collectives for the rocm backend, at one GPU.

The surface is the CUDA backend's ``__all__`` (difflet/backends/cuda/ops_impl/collectives.py:
213-241) with the CPU backend's world-size-1 semantics (difflet/backends/cpu/ops_impl/
collectives.py): every collective returns its input (or this rank's local slice, which at
world size 1 is the whole tensor), the rank helpers return 0 and the groups have size 1.

This build runs one process per GPU on one GPU. A process group of more than one rank (a
torchrun launch with WORLD_SIZE > 1) makes the group-taking collectives raise
NotImplementedError rather than silently skip the exchange; how the step would shard over
RCCL / xGMI is a design, not code, in this build.
"""

from __future__ import annotations

import os

import torch

_MULTI = ("multi-GPU collectives are not implemented on the rocm backend (this build runs one "
          "GPU: tp = cp = cfg = 1)")


class _SingleProcessGroup:
    def size(self):
        return 1

    def rank(self):
        return 0


class SPMDRank:
    """The rank as a (trace-friendly) module attribute; 0 at world size 1."""

    def __init__(self, world_size: int = 1):
        self.world_size = int(world_size)
        self.rank = torch.zeros(1, dtype=torch.int32)

    def get_rank(self):
        return self.rank


def _world_size() -> int:
    if torch.distributed.is_available() and torch.distributed.is_initialized():
        return torch.distributed.get_world_size()
    return int(os.environ.get("WORLD_SIZE", "1"))


def _single(what: str):
    if _world_size() > 1:
        raise NotImplementedError(f"{what}: {_MULTI}")


def gather_tp_dim(tensor, *, dim: int):
    _single("gather_tp_dim")
    return tensor


def gather_from_tensor_model_parallel_region_with_dim(tensor, gather_dim: int, process_group=None):
    if process_group is not None and _size(process_group) > 1:
        raise NotImplementedError(f"gather_from_tensor_model_parallel_region_with_dim: {_MULTI}")
    return tensor


def reduce_tp(tensor):
    _single("reduce_tp")
    return tensor


def reduce_from_tensor_model_parallel_region(tensor, process_group=None):
    if process_group is not None and _size(process_group) > 1:
        raise NotImplementedError(f"reduce_from_tensor_model_parallel_region: {_MULTI}")
    return tensor


def scatter_tp_dim(tensor, *, dim: int):
    _single("scatter_tp_dim")
    return tensor


def scatter_to_tensor_model_parallel_region(tensor, dim: int = -1):
    return scatter_tp_dim(tensor, dim=dim)


def scatter_to_process_group_spmd(tensor, *args, process_group=None, **kwargs):
    if process_group is not None and _size(process_group) > 1:
        raise NotImplementedError(f"scatter_to_process_group_spmd: {_MULTI}")
    return tensor


def scatter_to_sequence_parallel_region(tensor, *, dim: int):
    _single("scatter_to_sequence_parallel_region")
    return tensor


def gather_from_sequence_parallel_region(tensor, *, dim: int):
    _single("gather_from_sequence_parallel_region")
    return tensor


def reduce_scatter_to_sequence_parallel_region(tensor, *, dim: int):
    _single("reduce_scatter_to_sequence_parallel_region")
    return tensor


def _size(group) -> int:
    if isinstance(group, (list, tuple)):
        return len(group[0]) if group else 1
    if hasattr(group, "size"):
        return int(group.size())
    return 1


# ------------------------------------------------------------------ mesh (all axes size 1)
class _MeshSpec:
    dp = cfg = cp = tp = 1


_MESH = _MeshSpec()


def init_parallel_mesh(config=None):
    """Accepts a config whose parallel degrees are all 1; anything larger raises."""
    for axis in ("tp_degree", "cp_degree", "cfg_degree", "dp_degree", "world_size"):
        value = getattr(config, axis, 1) if config is not None else 1
        try:
            value = int(value)
        except (TypeError, ValueError):
            value = 1
        if value > 1:
            raise NotImplementedError(f"init_parallel_mesh: {axis}={value}: {_MULTI}")
    _single("init_parallel_mesh")
    return _MESH


def destroy_parallel_mesh():
    return None


def get_mesh_spec():
    return _MESH


def get_world_group():
    return _SingleProcessGroup()


def get_cfg_group():
    return _SingleProcessGroup()


def get_cp_group():
    return _SingleProcessGroup()


def get_cp_mesh():
    return _SingleProcessGroup()


def get_tp_groups():
    return [[0]]


def axis_replica_groups(axis: str):
    return [[0]]


def get_axis_rank(axis: str, global_rank=0) -> int:
    return 0


def get_tp_rank() -> int:
    return 0


def get_tp_size() -> int:
    return 1


def get_tensor_model_parallel_rank() -> int:
    return 0


def get_tensor_model_parallel_size() -> int:
    return 1


def get_cfg_rank_spmd(global_rank):
    return torch.zeros_like(global_rank) if isinstance(global_rank, torch.Tensor) else 0


def get_cp_rank_spmd(global_rank):
    return torch.zeros_like(global_rank) if isinstance(global_rank, torch.Tensor) else 0


__all__ = [
    "SPMDRank",
    "axis_replica_groups",
    "destroy_parallel_mesh",
    "gather_from_sequence_parallel_region",
    "gather_from_tensor_model_parallel_region_with_dim",
    "gather_tp_dim",
    "get_axis_rank",
    "get_cfg_group",
    "get_cfg_rank_spmd",
    "get_cp_group",
    "get_cp_mesh",
    "get_cp_rank_spmd",
    "get_mesh_spec",
    "get_tensor_model_parallel_rank",
    "get_tensor_model_parallel_size",
    "get_tp_groups",
    "get_tp_rank",
    "get_tp_size",
    "get_world_group",
    "init_parallel_mesh",
    "reduce_from_tensor_model_parallel_region",
    "reduce_scatter_to_sequence_parallel_region",
    "reduce_tp",
    "scatter_to_process_group_spmd",
    "scatter_to_sequence_parallel_region",
    "scatter_to_tensor_model_parallel_region",
    "scatter_tp_dim",
]
