"""``torch.compile`` for the rocm backend: per-block compilation of a DiT's repeated blocks, the
GPU backend's scheme (difflet/backends/gpu/application.py:53,60-81,148-166).

Each block of each repeated list is replaced by its ``torch.compile`` wrapper, so one graph
serves the whole stack and the module around the blocks stays eager. The HIP kernels reach the
graph as ``difflet_rocm::*`` custom operators (ops_impl/library.py), opaque nodes with fake
implementations, so a block that calls the op modules traces without a graph break and Inductor
compiles only the torch code between the kernels.
"""

from __future__ import annotations

from collections.abc import Iterable
from typing import Any

import torch
import torch.nn as nn

#: difflet/backends/gpu/application.py:53
COMPILE_MODE = "max-autotune-no-cudagraphs"

#: The repeated block lists by their diffusers attribute names, per model family
#: (difflet/backends/cuda/{flux,hunyuan_video,wan,ltx_2}/transformer.py repeated_blocks).
REPEATED_BLOCK_ATTRS: tuple[str, ...] = ("transformer_blocks", "single_transformer_blocks",
                                         "blocks")


def compile_blocks(block_lists: Iterable[nn.ModuleList], *, dynamic: bool,
                   options: dict[str, Any] | None = None, mode: str | None = COMPILE_MODE) -> int:
    """Replace every block of each list with its ``torch.compile`` wrapper, in place; returns
    how many were compiled (difflet/backends/gpu/application.py:60-81). ``options`` are added
    to the mode's own Inductor settings rather than replacing them."""
    if options is None:
        kwargs: dict[str, Any] = {"mode": mode}
    else:
        base = torch._inductor.list_mode_options(mode) if mode else {}
        kwargs = {"options": {**base, **options}}
    count = 0
    for blocks in block_lists:
        for i, block in enumerate(blocks):
            blocks[i] = torch.compile(block, dynamic=dynamic, fullgraph=False, **kwargs)
            count += 1
    return count


def repeated_blocks(module: nn.Module) -> list[nn.ModuleList]:
    """The module's repeated block lists: FLUX / HunyuanVideo ``transformer_blocks`` and
    ``single_transformer_blocks``, Qwen-Image ``transformer_blocks``, Wan ``blocks``; also one
    level down (LTX-2 keeps them under ``transformer``)."""
    found = [getattr(module, a) for a in REPEATED_BLOCK_ATTRS
             if isinstance(getattr(module, a, None), nn.ModuleList)]
    if not found and isinstance(getattr(module, "transformer", None), nn.Module):
        return repeated_blocks(module.transformer)
    return found


def compile_repeated_blocks_(module: nn.Module, *, dynamic: bool = False,
                             options: dict[str, Any] | None = None,
                             mode: str | None = COMPILE_MODE) -> int:
    """What the GPU component does with ``torch_compile`` set, after the weights are loaded and
    the load-time swaps are applied (difflet/backends/gpu/application.py:148-166)."""
    lists = repeated_blocks(module)
    if not lists:
        raise ValueError(f"{type(module).__name__} has none of the repeated block lists "
                         f"{REPEATED_BLOCK_ATTRS}")
    return compile_blocks(lists, dynamic=dynamic, options=options, mode=mode)


__all__ = ["COMPILE_MODE", "REPEATED_BLOCK_ATTRS", "compile_blocks", "compile_repeated_blocks_",
           "repeated_blocks"]
