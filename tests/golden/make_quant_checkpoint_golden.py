"""Writes quant_checkpoint_golden.json: what the reference's own quantized-checkpoint writer
(difflet/quant/checkpoint.py:325-392) and MX quantizer (difflet/quant/mx.py:96-108) produce on
the toy FLUX directory of quant_toy.py and on seeded rows at the awkward K values.

Run in a container that holds the reference at /root/reference (it is imported from there, torch
only); the JSON it writes is the fixture, and nothing else of the reference is kept:

    python tests/golden/make_quant_checkpoint_golden.py

Recorded per spec: the source fingerprint, the directory digest, the spec's dict, weights
identity and (compute "dequant") cache fields, the manifest without its time stamp and source
path, the index's weight map (shard file per key) and [dtype, shape, sha256] of every tensor the
writer stored."""

from __future__ import annotations

import dataclasses
import json
import sys
import tempfile
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
if str(HERE.parent.parent) not in sys.path:
    sys.path.insert(0, str(HERE.parent.parent))

from tests.golden.quant_toy import tensor_digest, write_toy_flux  # noqa: E402

AWKWARD_K = (384, 768, 896, 3456, 13824)
AWKWARD_ROWS = 4
SHARD_BYTES = 1 << 20
AWKWARD_TARGETS = (r"context_embedder", r"time_text_embed\.text_embedder\.linear_1",
                   r"transformer_blocks\.\d+\.attn\.(to_q|to_k)")


def awkward_rows(k: int) -> np.ndarray:
    """[4, k] fp32: N(0, 1) rows scaled by 1e-3, 1, 1e3 and 1e-36 (a row whose blocks all take
    the smallest E8M0 scale)."""
    rng = np.random.Generator(np.random.PCG64(7000 + k))
    x = rng.standard_normal((AWKWARD_ROWS, k), dtype=np.float32)
    x *= np.array([1e-3, 1.0, 1e3, 1e-36], dtype=np.float32)[:, None]
    return x


def main() -> None:
    # only a direct run of this script touches the reference (the tests import the helpers above)
    sys.path.insert(0, "/root/reference")
    from safetensors import safe_open

    from difflet.backends._torch_megatron.checkpoint import build_weight_map
    from difflet.quant import mx
    from difflet.quant.checkpoint import quantized_digest, source_fingerprint, write_quantized_dir
    from difflet.quant.spec import QuantSpec
    from difflet.quant.targets import default_spec

    specs = {"flux_mx": default_spec("flux"),
             "awkward_mx": QuantSpec(targets=AWKWARD_TARGETS, compute="dequant")}
    out: dict = {"shard_bytes": SHARD_BYTES, "specs": {}, "mx_awkward_k": {}}
    with tempfile.TemporaryDirectory() as tmp:
        src = write_toy_flux(tmp)
        fingerprint = source_fingerprint(src)
        out["fingerprint"] = fingerprint
        for label, spec in specs.items():
            qdir = Path(tmp) / f"q-{label}"
            manifest = write_quantized_dir(src, qdir, spec, shard_bytes=SHARD_BYTES)
            manifest.pop("written")
            manifest["source"].pop("path")
            weight_map = build_weight_map(qdir)
            tensors = {}
            for key, path in sorted(weight_map.items()):
                with safe_open(path, framework="pt") as handle:
                    tensors[key] = tensor_digest(handle.get_tensor(key))
            index = json.loads((qdir / "diffusion_pytorch_model.safetensors.index.json").read_text())
            out["specs"][label] = {
                "spec": spec.to_dict(),
                "weights_identity": spec.weights_identity(),
                "cache_fields_dequant": dataclasses.replace(spec, compute="dequant").cache_fields(),
                "digest": quantized_digest(spec, fingerprint),
                "manifest": manifest,
                "index_weight_map": index["weight_map"],
                "index_total_size": index["metadata"]["total_size"],
                "tensors": tensors,
                "copied_files": sorted(p.name for p in qdir.iterdir()
                                       if not p.name.endswith((".safetensors", ".json"))),
            }
    out["default_specs"] = {m: default_spec(m).to_dict() for m in ("flux", "qwen_image", "wan")}
    for k in AWKWARD_K:
        q, s = mx.quantize_mx(torch.from_numpy(awkward_rows(k)))
        out["mx_awkward_k"][str(k)] = {"codes": tensor_digest(q), "scales": tensor_digest(s)}
    (HERE / "quant_checkpoint_golden.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print("wrote", HERE / "quant_checkpoint_golden.json")


if __name__ == "__main__":
    main()
