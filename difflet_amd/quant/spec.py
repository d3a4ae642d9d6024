"""What is quantized and how, for the rocm backend. Torch-free.

The rocm twin of difflet/quant/spec.py's QuantSpec (:46-176): the same fields, matching,
serialisation and cache-key rules, plus

* the ``rocm`` compute mode (the HIP fp8 GEMMs) next to ``dequant`` (weights dequantized once
  to bf16, bf16 GEMM: memory-only);
* a ``format`` field: ``mxfp8`` (the reference's one format: e4m3 with one E8M0 scale per 32
  values along K, difflet/quant/mx.py) or ``fp8_rowwise`` (new in this build: e4m3 weights with
  one fp32 scale per output channel, activations quantized per token at run time;
  include/difflet_rocm.h difflet_rocm_quantize_fp8_rowwise states the law).

The cache and weight identities are the reference's dicts, whose ``quant`` field names the
format: ``"mxfp8"`` as the reference writes it, so keys and directory digests of existing specs
stay byte-identical, and ``"fp8_rowwise"`` for the new format, so its artifacts never collide.
"""

from __future__ import annotations

import dataclasses
import hashlib
import json
import re
from collections.abc import Iterable
from typing import Any

QUANT_SCHEMA = 3  # difflet/quant/spec.py:27
FORMATS = ("mxfp8", "fp8_rowwise")
COMPUTE_MODES = ("rocm", "dequant")
DEFAULT_COMPUTE = "rocm"
BLOCK = 32          # difflet/quant/spec.py:39
LAYOUT_K = 128      # difflet/quant/spec.py:40
STRIPPED_PREFIXES = ("transformer.",)


def strip_prefix(name: str) -> str:
    for prefix in STRIPPED_PREFIXES:
        if name.startswith(prefix):
            return name[len(prefix):]
    return name


@dataclasses.dataclass(frozen=True)
class RocmQuantSpec:
    targets: tuple[str, ...]
    compute: str = DEFAULT_COMPUTE
    tp_degree: int = 1
    row_parallel: tuple[str, ...] = ()
    split_linears: tuple[str, ...] = ()
    schema: int = QUANT_SCHEMA
    format: str = "mxfp8"

    def __post_init__(self) -> None:
        if int(self.tp_degree) != 1:
            raise ValueError(f"the rocm backend runs tp = 1, got tp_degree={self.tp_degree}")
        if self.compute not in COMPUTE_MODES:
            raise ValueError(f"compute must be one of {COMPUTE_MODES}, got {self.compute!r}")
        if self.format not in FORMATS:
            raise ValueError(f"format must be one of {FORMATS}, got {self.format!r}")
        if not self.targets or any(not t for t in self.targets):
            raise ValueError("a QuantSpec needs at least one non-empty target pattern")
        for pattern in (*self.targets, *self.row_parallel, *self.split_linears):
            re.compile(pattern)

    # ------------------------------------------------------------------ matching
    def matches(self, name: str) -> bool:
        bare = strip_prefix(name)
        return any(re.fullmatch(p, bare) for p in self.targets)

    def unmatched_targets(self, names: Iterable[str]) -> list[str]:
        bare = [strip_prefix(n) for n in names]
        return [p for p in self.targets if not any(re.fullmatch(p, n) for n in bare)]

    def is_row_parallel(self, name: str) -> bool:
        bare = strip_prefix(name)
        return any(re.fullmatch(p, bare) for p in self.row_parallel)

    def k_shards(self, name: str) -> int:
        return 1  # tp = 1

    def is_split(self, name: str) -> bool:
        bare = strip_prefix(name)
        return any(re.fullmatch(p, bare) for p in self.split_linears)

    def unmatched_splits(self, names: Iterable[str]) -> list[str]:
        """The split patterns that match none of ``names`` (difflet/quant/spec.py:113-119)."""
        bare = [strip_prefix(n) for n in names]
        return [p for p in self.split_linears if not any(re.fullmatch(p, n) for n in bare)]

    # ------------------------------------------------------------- serialisation
    def to_dict(self) -> dict[str, Any]:
        body = dataclasses.asdict(self)
        body["targets"] = list(self.targets)
        body["row_parallel"] = list(self.row_parallel)
        if self.split_linears:
            body["split_linears"] = list(self.split_linears)
        else:
            del body["split_linears"]
        return body

    @classmethod
    def from_dict(cls, body: dict[str, Any]) -> "RocmQuantSpec":
        body = dict(body)
        body["targets"] = tuple(body["targets"])
        body["row_parallel"] = tuple(body.get("row_parallel", ()))
        body["split_linears"] = tuple(body.get("split_linears", ()))
        body.setdefault("format", "mxfp8")
        return cls(**body)

    def targets_sha256(self) -> str:
        return hashlib.sha256(json.dumps(list(self.targets)).encode()).hexdigest()[:16]

    def cache_fields(self) -> dict[str, Any]:
        """difflet/quant/spec.py:147-157; ``quant`` is the format name."""
        fields = {
            "quant": self.format,
            "quant_schema": self.schema,
            "quant_compute": self.compute,
            "quant_targets_sha256": self.targets_sha256(),
            "quant_tp_degree": int(self.tp_degree),
        }
        return fields

    def weights_identity(self) -> dict[str, Any]:
        identity = {
            "quant": self.format,
            "quant_schema": self.schema,
            "quant_targets": list(self.targets),
            "quant_row_parallel": list(self.row_parallel),
            "quant_tp_degree": int(self.tp_degree),
        }
        if self.split_linears:
            identity["quant_split_linears"] = list(self.split_linears)
        return identity


_BLOCK = r"transformer_blocks\.\d+"
_SINGLE = r"single_transformer_blocks\.\d+"

#: Every linear of the FLUX blocks but the adaLN ones (the "every block linear" fp8 step);
#: diffusers' names, the single blocks' proj_out as the one fused [attn | mlp] linear.
FLUX_ALL_BLOCK_LINEARS: tuple[str, ...] = (
    rf"{_BLOCK}\.attn\.(to_q|to_k|to_v|add_q_proj|add_k_proj|add_v_proj|to_out\.0|to_add_out)",
    rf"{_BLOCK}\.(ff|ff_context)\.net\.(0\.proj|2)",
    rf"{_SINGLE}\.attn\.(to_q|to_k|to_v)",
    rf"{_SINGLE}\.(proj_mlp|proj_out)",
)

#: difflet/quant/targets.py:158 (SINGLE_BLOCK_SPLIT_LINEARS): the single blocks' proj_out, stored
#: by an mxfp8 checkpoint as proj_out_attn [D, D] and proj_out_mlp [D, 4D].
SINGLE_BLOCK_SPLIT_LINEARS: tuple[str, ...] = (rf"{_SINGLE}\.proj_out",)

#: difflet/quant/targets.py:162-169 (FLUX_TARGETS), the reference's default FLUX MXFP8 set: both
#: streams' q/k/v and MLPs, the single blocks' q/k/v, proj_mlp and both proj_out halves; the
#: double blocks' output projections stay bf16.
FLUX_MX_TARGETS: tuple[str, ...] = (
    rf"{_BLOCK}\.attn\.(to_q|to_k|to_v|add_q_proj|add_k_proj|add_v_proj)",
    rf"{_BLOCK}\.(ff|ff_context)\.net\.0\.proj",
    rf"{_BLOCK}\.(ff|ff_context)\.net\.2",
    rf"{_SINGLE}\.attn\.(to_q|to_k|to_v)",
    rf"{_SINGLE}\.proj_mlp",
    rf"{_SINGLE}\.proj_out_(attn|mlp)",
)

#: difflet/quant/targets.py:189-193 (FLUX_ROW_PARALLEL). It changes no byte at tp = 1 but is part
#: of the spec's weights identity, so a spec that names it keeps the reference's digest.
FLUX_ROW_PARALLEL: tuple[str, ...] = (
    rf"{_BLOCK}\.attn\.(to_out\.0|to_add_out)",
    rf"{_BLOCK}\.(ff|ff_context)\.net\.2",
    rf"{_SINGLE}\.proj_out_(attn|mlp)",
)

#: difflet/quant/targets.py:259-263 (WAN_TARGETS), on diffusers' checkpoint names: the
#: cross-attention's q/k/v and both FFN linears.
WAN_TARGETS: tuple[str, ...] = (
    r"blocks\.\d+\.attn2\.(to_q|to_k|to_v)",
    r"blocks\.\d+\.ffn\.net\.0\.proj",
    r"blocks\.\d+\.ffn\.net\.2",
)

#: difflet/quant/targets.py:117-121 (QWEN_IMAGE_TARGETS): q/k/v, the added q/k/v and both MLPs;
#: the output projections stay bf16.
QWEN_IMAGE_TARGETS: tuple[str, ...] = (
    rf"{_BLOCK}\.attn\.(to_q|to_k|to_v|add_q_proj|add_k_proj|add_v_proj)",
    rf"{_BLOCK}\.(img_mlp|txt_mlp)\.net\.0\.proj",
    rf"{_BLOCK}\.(img_mlp|txt_mlp)\.net\.2",
)

#: difflet/quant/targets.py:138-141 (QWEN_IMAGE_ROW_PARALLEL)
QWEN_IMAGE_ROW_PARALLEL: tuple[str, ...] = (
    rf"{_BLOCK}\.attn\.(to_out\.0|to_add_out)",
    rf"{_BLOCK}\.(img_mlp|txt_mlp)\.net\.2",
)

#: difflet/quant/targets.py:278-281 (WAN_ROW_PARALLEL)
WAN_ROW_PARALLEL: tuple[str, ...] = (
    r"blocks\.\d+\.(attn1|attn2)\.to_out\.0",
    r"blocks\.\d+\.ffn\.net\.2",
)

#: difflet/quant/targets.py:376-397: the MXFP8 recipe of each model family this backend runs
TARGETS_BY_MODEL = {"flux": FLUX_MX_TARGETS, "qwen_image": QWEN_IMAGE_TARGETS, "wan": WAN_TARGETS}
ROW_PARALLEL_BY_MODEL = {"flux": FLUX_ROW_PARALLEL, "qwen_image": QWEN_IMAGE_ROW_PARALLEL,
                         "wan": WAN_ROW_PARALLEL}
SPLITS_BY_MODEL = {"flux": SINGLE_BLOCK_SPLIT_LINEARS}


def _onto_fused(patterns: tuple[str, ...], splits: tuple[str, ...]) -> tuple[str, ...]:
    """``patterns`` with each name of a split linear's stored halves (``<split>_(attn|mlp)``)
    turned back into the fused linear's name ``<split>``, duplicates dropped."""
    halves = {rf"{sp}_(attn|mlp)": sp for sp in splits}
    out: list[str] = []
    for pat in patterns:
        pat = halves.get(pat, pat)
        if pat not in out:
            out.append(pat)
    return tuple(out)


def default_spec(model: str, **overrides) -> RocmQuantSpec:
    """difflet/quant/targets.py:424-440: the model's MXFP8 recipe (targets, row-parallel and split
    linears as the reference names them, so the quantized directory's digest is the reference's);
    ``targets=``, ``compute=`` and ``format=`` override. A per-channel fp8 spec keeps the fused
    linears (no splits), since one scale per output channel spans the whole K: patterns that
    name a split linear's halves name the fused linear instead."""
    if model not in TARGETS_BY_MODEL:
        raise ValueError(f"no fp8 target layers are defined for {model!r}; models with fp8 "
                         f"support: {sorted(TARGETS_BY_MODEL)}")
    splits = SPLITS_BY_MODEL.get(model, ())
    row_parallel = ROW_PARALLEL_BY_MODEL.get(model, ())
    targets = TARGETS_BY_MODEL[model]
    if overrides.get("format", "mxfp8") == "mxfp8":
        overrides.setdefault("split_linears", splits)
    else:
        row_parallel, targets = _onto_fused(row_parallel, splits), _onto_fused(targets, splits)
    overrides.setdefault("row_parallel", row_parallel)
    overrides.setdefault("targets", targets)
    return RocmQuantSpec(**overrides)
