"""Writes attention_reference.json: the reference CPU backend's attention op
(difflet/backends/cpu/ops_impl/attention.py:8-48) on seeded inputs, for every form of the
attention contract (plain, scale None, causal, bool and additive masks with a fully masked row,
per-query key bounds, the (B*H, S, D) layout), in fp32 and bf16.

Run in a container that holds the reference at /root/reference (imported from there; the JSON it
writes is the fixture, nothing else of the reference is kept):

    python tests/golden/make_attention_golden.py
"""

from __future__ import annotations

import base64
import json
import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
if str(HERE.parent.parent) not in sys.path:
    sys.path.insert(0, str(HERE.parent.parent))

B, H, SQ, SK, D = 1, 2, 7, 9, 128


def _rand(rng, shape, scale=1.0):
    return torch.from_numpy(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))


def cases(dtype: torch.dtype) -> dict[str, tuple[tuple, dict]]:
    """name -> ((q, k, v), kwargs) for the attention op; inputs are rounded to `dtype`."""
    rng = np.random.Generator(np.random.PCG64(4242))
    q, k, v = (_rand(rng, (B, H, n, D)).to(dtype) for n in (SQ, SK, SK))
    sq = _rand(rng, (B, H, SK, D)).to(dtype)  # a square query set for the causal case
    bool_mask = torch.from_numpy(rng.random((B, H, SQ, SK)) < 0.6)
    bool_mask[0, 1, 3] = False  # a fully masked row: it averages v
    add_mask = _rand(rng, (B, 1, SQ, SK), 2.0).to(dtype)
    bmin = torch.from_numpy(rng.integers(0, 4, (B * H, SQ, 1)).astype(np.int32))
    bmax = bmin + torch.from_numpy(rng.integers(1, SK - 3, (B * H, SQ, 1)).astype(np.int32))
    fold = lambda t: t.reshape(B * H, t.shape[2], D)  # noqa: E731
    return {
        "plain": ((q, k, v), {"scale": 0.25}),
        "scale_none": ((q, k, v), {}),
        "causal": ((sq, k, v), {"scale": 0.25, "causal": True}),
        "bool_mask": ((q, k, v), {"scale": 0.25, "attention_mask": bool_mask}),
        "additive_mask": ((q, k, v), {"scale": 0.25, "attention_mask": add_mask}),
        "bounds_folded": ((fold(q), fold(k), fold(v)),
                          {"scale": 0.5, "bound_min": bmin, "bound_max": bmax}),
    }


def encode(t: torch.Tensor) -> dict:
    return {"shape": list(t.shape),
            "f32": base64.b64encode(t.float().contiguous().numpy().astype("<f4").tobytes()).decode()}


def decode(rec: dict) -> torch.Tensor:
    raw = np.frombuffer(base64.b64decode(rec["f32"]), dtype="<f4").copy()
    return torch.from_numpy(raw).reshape(rec["shape"])


def main() -> None:
    # only a direct run of this script touches the reference (the tests import the helpers above)
    sys.path.insert(0, "/root/reference")
    os.environ["DIFFLET_BACKEND"] = "cpu"
    from difflet.backends.cpu.ops_impl.attention import attention

    out = {}
    for dtype in (torch.float32, torch.bfloat16):
        for name, ((q, k, v), kw) in cases(dtype).items():
            y = attention(q, k, v, **kw)
            out[f"{name}.{str(dtype).removeprefix('torch.')}"] = encode(y)
    (HERE / "attention_reference.json").write_text(json.dumps(out, indent=0) + "\n")
    print("wrote", HERE / "attention_reference.json", len(out))


if __name__ == "__main__":
    main()
