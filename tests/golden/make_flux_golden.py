"""Writes flux_reference_forward.json: the output of the reference's own FLUX transformer
(difflet/models/flux/modeling_flux.py:219-613, NeuronFluxTransformer2DModel on the reference's
CPU backend, fp32) for the oracle's seeded weights and inputs at a small FLUX shape: hidden 256
(2 heads of 128), 2 double + 2 single blocks, a 4 x 4 patch grid and 8 text tokens.

Run in a container that holds the reference at /root/reference (imported from there; the XLA
module-boundary markers are replaced by identities, as the reference's own CPU tests do in
tests/unit/models/flux/test_flux_modeling.py:60-75):

    python tests/golden/make_flux_golden.py

The JSON holds the output and the reference's outputs after the first double block (both
streams) and the first single block ([txt | img] rows), as fp32 bytes; nothing of the reference
is kept."""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
if str(HERE.parent.parent) not in sys.path:
    sys.path.insert(0, str(HERE.parent.parent))

from oracle import flux as oflux  # noqa: E402
from oracle import ops  # noqa: E402

SHAPE = oflux.FluxShape(hidden=256, heads=2, head_dim=128, n_double=2, n_single=2,
                        in_channels=16, out_channels=16, txt_dim=64, pooled_dim=32)
SEED, IMG_HW, TXT = 5, (4, 4), 8


def oracle_state_dict() -> dict:
    """Every parameter of the oracle's draw under its diffusers name, fp32."""
    sd = dict(oflux.embed_weights(SHAPE, SEED, dtype=torch.float32))
    for i in range(SHAPE.n_double):
        for k, v in oflux.double_block_weights(SHAPE, SEED, i, dtype=torch.float32).items():
            sd[k if k.startswith("transformer_blocks.") else f"transformer_blocks.{i}.{k}"] = v
    for i in range(SHAPE.n_single):
        for k, v in oflux.single_block_weights(SHAPE, SEED, i, dtype=torch.float32).items():
            sd[k if k.startswith("single_transformer_blocks.") else f"single_transformer_blocks.{i}.{k}"] = v
    return sd


def encode(t: torch.Tensor) -> str:
    import base64

    return base64.b64encode(t.detach().float().contiguous().numpy().astype("<f4").tobytes()).decode()


def decode(rec: dict) -> torch.Tensor:
    import base64

    import numpy as np

    raw = np.frombuffer(base64.b64decode(rec["f32"]), dtype="<f4").copy()
    return torch.from_numpy(raw).reshape(rec["shape"])


def inputs() -> dict:
    return oflux.synthetic_inputs(SHAPE, SEED, IMG_HW, TXT)


def main() -> None:
    # only a direct run of this script touches the reference (the tests import the helpers above)
    sys.path.insert(0, "/root/reference")
    os.environ["DIFFLET_BACKEND"] = "cpu"
    os.environ.setdefault("NEURON_PLATFORM_TARGET_OVERRIDE", "trn2")
    import difflet.layers.normalization as norm_mod
    import difflet.models.flux.modeling_flux as mf
    from difflet.models.flux.dit_config import FluxDiTConfig

    ident = lambda *a: a[0] if len(a) == 1 else a  # noqa: E731
    for mod in (mf, norm_mod):
        mod.ModuleMarkerStartWrapper = lambda: ident
        mod.ModuleMarkerEndWrapper = lambda: ident
    cfg = FluxDiTConfig(torch_dtype=torch.float32, attention_head_dim=SHAPE.head_dim,
                        guidance_embeds=True, in_channels=SHAPE.in_channels,
                        joint_attention_dim=SHAPE.txt_dim, num_attention_heads=SHAPE.heads,
                        num_layers=SHAPE.n_double, num_single_layers=SHAPE.n_single,
                        patch_size=1, pooled_projection_dim=SHAPE.pooled_dim, height=16, width=16,
                        out_channels=SHAPE.out_channels)
    model = mf.NeuronFluxTransformer2DModel(cfg).eval().to(torch.float32)
    sd = oracle_state_dict()
    d = SHAPE.hidden
    for i in range(SHAPE.n_single):
        # the model runs proj_out as its two column ranges, the bias on the attention half
        p = f"single_transformer_blocks.{i}.proj_out"
        w, b = sd.pop(f"{p}.weight"), sd.pop(f"{p}.bias")
        sd[f"{p}_attn.weight"], sd[f"{p}_attn.bias"] = w[:, :d].contiguous(), b
        sd[f"{p}_mlp.weight"] = w[:, d:].contiguous()
    missing, unexpected = model.load_state_dict(sd, strict=False)
    params = {n for n, _ in model.named_parameters()}
    missing = [m for m in missing if m in params]
    if missing or unexpected:
        raise SystemExit(f"name mismatch: missing {missing[:8]}, unexpected {unexpected[:8]}")
    inp = inputs()
    cos, sin = ops.flux_pos_embed(ops.flux_ids(TXT, *IMG_HW), SHAPE.axes)
    rot = torch.stack([cos, sin], dim=-1)
    seen = {}

    def keep(name):
        def hook(_m, _args, out):
            seen.setdefault(name, out)
        return hook

    model.transformer_blocks[0].register_forward_hook(keep("double0"))
    model.single_transformer_blocks[0].register_forward_hook(keep("single0"))
    with torch.no_grad():
        out = model(hidden_states=inp["latents"], encoder_hidden_states=inp["text"],
                    pooled_projections=inp["pooled"], timestep=inp["timestep"],
                    guidance=inp["guidance"], image_rotary_emb=rot)
    out = out[0] if isinstance(out, tuple) else out
    enc0, hid0 = seen["double0"]
    single0 = seen["single0"]
    single0 = single0[0] if isinstance(single0, tuple) else single0
    rec = {
        "shape": {k: (list(v) if isinstance(v, tuple) else v) for k, v in vars(SHAPE).items()},
        "seed": SEED, "img_hw": list(IMG_HW), "txt_len": TXT,
        "encoding": "base64 of little-endian float32, row-major",
        "tensors": {name: {"shape": list(t.shape), "f32": encode(t)} for name, t in
                    (("output", out), ("double0_context", enc0), ("double0_hidden", hid0),
                     ("single0", single0))},
    }
    (HERE / "flux_reference_forward.json").write_text(json.dumps(rec) + "\n")
    print("wrote", HERE / "flux_reference_forward.json", list(out.shape), list(single0.shape))


if __name__ == "__main__":
    main()
