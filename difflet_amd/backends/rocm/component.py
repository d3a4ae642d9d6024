"""What the rocm DiT components share: a lazy reader of a diffusers safetensors directory and
the component life cycle of the reference's GPU flow (difflet/backends/gpu/application.py:
build the module, load the weights, run `forward`), for a module that is one of the fused
steps of difflet_amd.dit.

The fused steps take every parameter through a `get(name)` callable as they build, so a
component needs no meta-device module and no state-dict copy: `SafetensorsDir.get` reads one
tensor at a time from the checkpoint files (a diffusers `transformer/` directory holds either
`diffusion_pytorch_model.safetensors` or an index plus shards), and the step moves it to the
device and concatenates it into its fused layout.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import torch


class SafetensorsDir:
    """The tensors of a safetensors directory (or one file) by name, read on demand. `prefix`
    is prepended to every name (the reference loads Qwen-Image under "transformer.",
    difflet/backends/cuda/qwen_image/transformer.py:22)."""

    def __init__(self, path, prefix: str = ""):
        self.path = Path(path)
        self.prefix = prefix
        from safetensors import safe_open

        self._where: dict[str, Path] = {}
        self._handles = {}
        idx = [] if self.path.is_file() else sorted(self.path.glob("*.safetensors.index.json"))
        if idx:  # an index names the shard of every tensor
            body = json.loads(idx[0].read_text())
            self._where = {name: self.path / shard for name, shard in body["weight_map"].items()}
            files = sorted(set(self._where.values()))
        else:
            files = [self.path] if self.path.is_file() else sorted(self.path.glob("*.safetensors"))
        if not files:
            raise FileNotFoundError(f"no safetensors files under {self.path}")
        for f in files:
            self._handles[f] = safe_open(str(f), framework="pt", device="cpu")
            if not idx:
                for name in self._handles[f].keys():
                    self._where.setdefault(name, f)

    def keys(self) -> list[str]:
        return sorted(self._where)

    def __contains__(self, name: str) -> bool:
        return self.prefix + name in self._where

    def get(self, name: str) -> torch.Tensor:
        key = self.prefix + name
        f = self._where.get(key)
        if f is None:
            raise KeyError(f"{key!r} is not in the checkpoint at {self.path}")
        return self._handles[f].get_tensor(key)

    __getitem__ = get


@dataclass
class Transformer2DModelOutput:
    """diffusers' output type (`sample`), for callers that read `.sample` when diffusers is
    not installed; with diffusers present its own class is used."""

    sample: torch.Tensor

    def __getitem__(self, i):
        return (self.sample,)[i]


def model_output(sample: torch.Tensor):
    try:
        from diffusers.models.modeling_outputs import Transformer2DModelOutput as _Out
    except ImportError:
        _Out = Transformer2DModelOutput
    return _Out(sample=sample)


class RocmComponent:
    """The life cycle a DiT component follows in the GPU flow: constructed from
    (model_path, config, device), `load()` builds the module with its weights on the device,
    `forward` / `__call__` runs it. `get` (a callable returning a parameter by name) replaces
    the checkpoint directory, for weights held elsewhere (tests, random weights).

    `torch_compile` is accepted for the reference's signature: the fused step is a fixed
    sequence of HIP launches with no torch graph to compile, so it changes nothing."""

    def __init__(self, *, model_path=None, config, device=None, torch_compile: bool = False,
                 get: Callable[[str], torch.Tensor] | None = None):
        if model_path is None and get is None:
            raise ValueError("a component needs model_path (a safetensors directory) or get")
        self.model_path = model_path
        self.dit_config = config
        self.dtype = getattr(config, "torch_dtype", torch.bfloat16)
        if self.dtype != torch.bfloat16:
            raise NotImplementedError(
                f"the rocm fused steps run bf16 activations, not {self.dtype}")
        self.device = torch.device(device if device is not None else "cuda")
        self.torch_compile = bool(torch_compile)
        self._get = get
        self.module = None

    @property
    def is_loaded(self) -> bool:
        return self.module is not None

    def weight_source(self, prefix: str = "") -> Callable[[str], torch.Tensor]:
        if self._get is not None:
            return self._get
        return SafetensorsDir(self.model_path, prefix).get

    def build_module(self):
        raise NotImplementedError

    def load(self, compiled_model_path=None, start_rank_id=None, local_ranks_size=None,
             skip_warmup: bool = False) -> None:
        """Builds the fused step on the device. The arguments of the reference's `load` are
        accepted; there is nothing compiled ahead of time to read."""
        del compiled_model_path, start_rank_id, local_ranks_size, skip_warmup
        if self.device.type != "cuda":
            raise RuntimeError(f"the rocm components run on a ROCm device, not {self.device}")
        from difflet_amd import _lib

        _lib.load()  # the kernels must be there; no fallback path
        self.module = self.build_module()

    def repeated_blocks(self, module=None) -> list:
        """No torch-compiled blocks: the fused step launches its kernels directly."""
        return []

    def _require_loaded(self):
        if self.module is None:
            raise RuntimeError("model is not loaded; call load() first")
        return self.module

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)


__all__ = ["RocmComponent", "SafetensorsDir", "Transformer2DModelOutput", "model_output"]
