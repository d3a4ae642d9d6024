"""A small diffusers-layout FLUX transformer directory, written deterministically (numpy PCG64
draws, bf16 by round-to-nearest-even, one fp32 tensor), for the quantized-checkpoint tests.

hidden 512 (4 heads of 128), MLP 2048, one double and one single block, text width 896 (an
MX K of one 512 tile plus a 384 remainder tile) and pooled width 384 (a remainder tile alone).
Two safetensors shards with an index, config.json and one more non-tensor file, as a hub
snapshot holds them. Edge rows: an all-zero row, a row scaled by 1e4 and one by 1e-30 (the
E8M0 scale's lower clamp) in the double block's to_q."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

TOY_SEED = 20261201
TOY_CONFIG = {
    "_class_name": "FluxTransformer2DModel",
    "attention_head_dim": 128,
    "axes_dims_rope": [16, 56, 56],
    "guidance_embeds": True,
    "in_channels": 64,
    "joint_attention_dim": 896,
    "num_attention_heads": 4,
    "num_layers": 1,
    "num_single_layers": 1,
    "out_channels": 64,
    "patch_size": 1,
    "pooled_projection_dim": 384,
}
D, F, HD = 512, 2048, 128
SHARD_FILES = ("diffusion_pytorch_model-00001-of-00002.safetensors",
               "diffusion_pytorch_model-00002-of-00002.safetensors")
INDEX = "diffusion_pytorch_model.safetensors.index.json"


def toy_shapes() -> dict[str, tuple[int, ...]]:
    out: dict[str, tuple[int, ...]] = {}

    def lin(name, o, i):
        out[f"{name}.weight"] = (o, i)
        out[f"{name}.bias"] = (o,)

    lin("x_embedder", D, 64)
    lin("context_embedder", D, 896)
    for e, i in (("timestep_embedder", 256), ("guidance_embedder", 256), ("text_embedder", 384)):
        lin(f"time_text_embed.{e}.linear_1", D, i)
        lin(f"time_text_embed.{e}.linear_2", D, D)
    lin("norm_out.linear", 2 * D, D)
    lin("proj_out", 64, D)
    p = "transformer_blocks.0"
    lin(f"{p}.norm1.linear", 6 * D, D)
    lin(f"{p}.norm1_context.linear", 6 * D, D)
    for n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_out.0",
              "to_add_out"):
        lin(f"{p}.attn.{n}", D, D)
    for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
        out[f"{p}.attn.{n}.weight"] = (HD,)
    lin(f"{p}.ff.net.0.proj", F, D)
    lin(f"{p}.ff.net.2", D, F)
    lin(f"{p}.ff_context.net.0.proj", F, D)
    lin(f"{p}.ff_context.net.2", D, F)
    p = "single_transformer_blocks.0"
    lin(f"{p}.norm.linear", 3 * D, D)
    lin(f"{p}.proj_mlp", F, D)
    for n in ("to_q", "to_k", "to_v"):
        lin(f"{p}.attn.{n}", D, D)
    for n in ("norm_q", "norm_k"):
        out[f"{p}.attn.{n}.weight"] = (HD,)
    lin(f"{p}.proj_out", D, D + F)
    return out


def toy_tensors() -> dict[str, torch.Tensor]:
    """Every tensor of the toy by name; the draw order is the sorted name order."""
    rng = np.random.Generator(np.random.PCG64(TOY_SEED))
    out: dict[str, torch.Tensor] = {}
    for name, shape in sorted(toy_shapes().items()):
        if ".norm_" in name:
            a = 1.0 + 0.1 * rng.standard_normal(shape, dtype=np.float32)
        else:
            a = 0.02 * rng.standard_normal(shape, dtype=np.float32)
        if name == "transformer_blocks.0.attn.to_q.weight":
            a[0] = 0.0
            a[1] *= 1e4
            a[2] *= 1e-30
        t = torch.from_numpy(a)
        out[name] = t if name.startswith("context_embedder.") else t.to(torch.bfloat16)
    return out


def write_toy_flux(root: str | Path) -> Path:
    """Write the toy into ``root/transformer`` and return that directory."""
    from safetensors.torch import save_file

    d = Path(root) / "transformer"
    d.mkdir(parents=True, exist_ok=True)
    tensors = toy_tensors()
    names = sorted(tensors)
    # the double block in the first file, everything else in the second
    first = [n for n in names if n.startswith("transformer_blocks.")]
    second = [n for n in names if n not in first]
    weight_map, total = {}, 0
    for fname, keys in zip(SHARD_FILES, (first, second)):
        save_file({k: tensors[k].contiguous() for k in keys}, str(d / fname),
                  metadata={"format": "pt"})
        for k in keys:
            weight_map[k] = fname
            total += tensors[k].numel() * tensors[k].element_size()
    index = {"metadata": {"total_size": total}, "weight_map": weight_map}
    (d / INDEX).write_text(json.dumps(index, indent=2, sort_keys=True) + "\n")
    (d / "config.json").write_text(json.dumps(TOY_CONFIG, indent=2, sort_keys=True) + "\n")
    (d / "README.txt").write_text("toy FLUX transformer for the quantized-checkpoint tests\n")
    return d


def tensor_digest(t: torch.Tensor) -> list:
    """[dtype, shape, sha256 of the bytes] of a CPU tensor."""
    import hashlib

    t = t.contiguous()
    raw = t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16 if t.element_size() == 2 else torch.int32)
    return [str(t.dtype).removeprefix("torch."), list(t.shape),
            hashlib.sha256(raw.numpy().tobytes()).hexdigest()]
