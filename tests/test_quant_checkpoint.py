"""The quantized-checkpoint host logic on the CPU: the directory's identity (fingerprint, digest,
path) against what the reference's own writer recorded on the same toy directory, the refusals
made before anything is quantized, the manifest check, the reader, and the MX oracle against the
reference's quantizer at the awkward K values. The quantizing writer itself needs the GPU
(test_gpu_quant_checkpoint.py)."""

from __future__ import annotations

import dataclasses
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from difflet_amd.quant import checkpoint as qc
from difflet_amd.quant.spec import (FLUX_ALL_BLOCK_LINEARS, FLUX_MX_TARGETS, FLUX_ROW_PARALLEL,
                                    SINGLE_BLOCK_SPLIT_LINEARS, RocmQuantSpec)
from oracle import mx as omx
from tests.golden.make_quant_checkpoint_golden import AWKWARD_K, AWKWARD_TARGETS, awkward_rows
from tests.golden.quant_toy import tensor_digest, write_toy_flux

GOLDEN = json.loads((Path(__file__).parent / "golden" / "quant_checkpoint_golden.json").read_text())


def ours(label: str, **kw) -> RocmQuantSpec:
    """Our spec with the fields of the reference spec the golden file records."""
    body = dict(GOLDEN["specs"][label]["spec"])
    body["compute"] = kw.pop("compute", "rocm")
    return dataclasses.replace(RocmQuantSpec.from_dict(body), **kw)


@pytest.fixture(scope="module")
def toy(tmp_path_factory):
    return write_toy_flux(tmp_path_factory.mktemp("toy"))


def test_reference_spec_fields_are_ours():
    flux = GOLDEN["specs"]["flux_mx"]["spec"]
    assert tuple(flux["targets"]) == FLUX_MX_TARGETS
    assert tuple(flux["row_parallel"]) == FLUX_ROW_PARALLEL
    assert tuple(flux["split_linears"]) == SINGLE_BLOCK_SPLIT_LINEARS
    assert tuple(GOLDEN["specs"]["awkward_mx"]["spec"]["targets"]) == AWKWARD_TARGETS
    for label in GOLDEN["specs"]:
        # to_dict round trip, compute aside (the reference's modes are its own)
        ref = dict(GOLDEN["specs"][label]["spec"])
        mine = ours(label).to_dict()
        assert {k: v for k, v in mine.items() if k != "compute"} == \
            {k: v for k, v in ref.items() if k != "compute"}


def test_fingerprint_digest_and_keys_equal_the_reference(toy, tmp_path):
    assert qc.source_fingerprint(toy) == GOLDEN["fingerprint"]
    for label, rec in GOLDEN["specs"].items():
        spec = ours(label)
        assert spec.weights_identity() == rec["weights_identity"]
        assert qc.quantized_digest(spec, qc.source_fingerprint(toy)) == rec["digest"]
        assert ours(label, compute="dequant").cache_fields() == rec["cache_fields_dequant"]
        path = qc.quantized_dir(tmp_path / "cache", toy, spec)
        assert path == (tmp_path / "cache" / "quantized" / toy.parent.name / "transformer"
                        / f"mxfp8-{rec['digest']}")


def test_fingerprint_ignores_mtimes_and_tracks_bytes(toy, tmp_path):
    import os
    import shutil

    copy = tmp_path / "copy" / "transformer"
    shutil.copytree(toy, copy)
    for p in copy.iterdir():
        os.utime(p, (0, 0))
    assert qc.source_fingerprint(copy) == GOLDEN["fingerprint"]
    shard = sorted(copy.glob("*.safetensors"))[0]
    shard.write_bytes(shard.read_bytes() + b"\0")
    assert qc.source_fingerprint(copy) != GOLDEN["fingerprint"]


def test_a_new_format_is_another_directory(toy):
    fp = qc.source_fingerprint(toy)
    mx = RocmQuantSpec(targets=FLUX_ALL_BLOCK_LINEARS)
    rw = RocmQuantSpec(targets=FLUX_ALL_BLOCK_LINEARS, format="fp8_rowwise")
    assert qc.quantized_digest(mx, fp) != qc.quantized_digest(rw, fp)
    assert rw.weights_identity()["quant"] == "fp8_rowwise"
    assert rw.cache_fields()["quant"] == "fp8_rowwise"


def test_hub_snapshot_label(tmp_path):
    snap = tmp_path / "hub" / "models--black-forest-labs--FLUX.1-dev" / "snapshots" / "0123456789abcdef" / "transformer"
    write_toy_flux(snap.parent)
    spec = RocmQuantSpec(targets=FLUX_ALL_BLOCK_LINEARS)
    path = qc.quantized_dir(tmp_path / "c", snap, spec)
    assert path.parts[-3] == "black-forest-labs--FLUX.1-dev__01234567"


@pytest.mark.parametrize("spec, message", [
    (RocmQuantSpec(targets=(r"no_such_linear",)), "target patterns match no linear weight"),
    (RocmQuantSpec(targets=(r"single_transformer_blocks\.\d+\.proj_out",),
                   split_linears=SINGLE_BLOCK_SPLIT_LINEARS),
     "name single_transformer_blocks.0.proj_out_attn / single_transformer_blocks.0.proj_out_mlp"),
    (RocmQuantSpec(targets=FLUX_MX_TARGETS, split_linears=(r"nothing\.here",)),
     "split patterns match no linear weight"),
    (RocmQuantSpec(targets=FLUX_MX_TARGETS, split_linears=SINGLE_BLOCK_SPLIT_LINEARS,
                   row_parallel=(r"single_transformer_blocks\.\d+\.proj_out",)),
     "row-parallel patterns name the fused weight"),
    (RocmQuantSpec(targets=FLUX_ALL_BLOCK_LINEARS, format="fp8_rowwise",
                   split_linears=SINGLE_BLOCK_SPLIT_LINEARS), "split_linears must be empty"),
])
def test_refusals_come_before_any_quantization(toy, tmp_path, spec, message):
    out = tmp_path / "q"
    with pytest.raises(ValueError, match=message.replace("(", r"\(").replace(".", r"\.")):
        qc.write_quantized_dir(toy, out, spec, device="cpu")
    assert not out.exists() and not list(tmp_path.glob(".q.tmp-*"))


def test_existing_directory_is_refused(toy, tmp_path):
    out = tmp_path / "q"
    out.mkdir()
    (out / qc.MANIFEST).write_text("{}")
    with pytest.raises(FileExistsError):
        qc.write_quantized_dir(toy, out, RocmQuantSpec(targets=FLUX_ALL_BLOCK_LINEARS), device="cpu")


def _fake_quantized(toy, out: Path, spec_body: dict, files=("a.safetensors",)) -> None:
    out.mkdir(parents=True)
    for f in files:
        (out / f).write_bytes(b"x")
    (out / qc.INDEX_NAME).write_text("{}")
    manifest = {"schema": 3, "spec": spec_body, "files": list(files),
                "source": {"fingerprint": qc.source_fingerprint(toy)}}
    (out / qc.MANIFEST).write_text(json.dumps(manifest))


def test_check_quantized_dir(toy, tmp_path):
    spec = ours("flux_mx")
    # a directory the reference wrote (its compute mode "nki") is accepted for the same bytes
    good = tmp_path / "good"
    _fake_quantized(toy, good, GOLDEN["specs"]["flux_mx"]["spec"])
    assert qc.check_quantized_dir(good, toy, spec)["schema"] == 3
    with pytest.raises(ValueError, match="never written"):
        qc.check_quantized_dir(tmp_path / "absent", toy, spec)
    with pytest.raises(ValueError, match="another quantization spec"):
        qc.check_quantized_dir(good, toy, ours("awkward_mx"))
    with pytest.raises(ValueError, match="another quantization spec"):
        qc.check_quantized_dir(good, toy, dataclasses.replace(spec, format="fp8_rowwise",
                                                              split_linears=()))
    bad_schema = tmp_path / "schema"
    _fake_quantized(toy, bad_schema, dict(GOLDEN["specs"]["flux_mx"]["spec"], schema=2))
    m = json.loads((bad_schema / qc.MANIFEST).read_text())
    m["schema"] = 2
    (bad_schema / qc.MANIFEST).write_text(json.dumps(m))
    with pytest.raises(ValueError, match="schema 2 != 3"):
        qc.check_quantized_dir(bad_schema, toy, spec)
    missing = tmp_path / "missing"
    _fake_quantized(toy, missing, GOLDEN["specs"]["flux_mx"]["spec"], files=("a.safetensors", "b.safetensors"))
    (missing / "b.safetensors").unlink()
    with pytest.raises(ValueError, match="b.safetensors is missing"):
        qc.check_quantized_dir(missing, toy, spec)
    other = tmp_path / "other" / "transformer"
    write_toy_flux(other.parent)
    shard = sorted(other.glob("*.safetensors"))[0]
    shard.write_bytes(shard.read_bytes() + b"\0")
    with pytest.raises(ValueError, match="another checkpoint"):
        qc.check_quantized_dir(good, other, spec)
    tp2 = tmp_path / "tp2"
    _fake_quantized(toy, tp2, dict(GOLDEN["specs"]["flux_mx"]["spec"], tp_degree=2))
    with pytest.raises(ValueError, match="another quantization spec"):
        qc.check_quantized_dir(tp2, toy, spec)
    with pytest.raises(ValueError, match="write it first"):
        qc.ensure_quantized_dir(tmp_path / "cache", toy, spec, create=False)


def test_reader_checks_scale_layout(tmp_path):
    from safetensors.torch import save_file

    d = tmp_path / "r"
    d.mkdir()
    w = torch.zeros(4, 128).to(torch.float8_e4m3fn)
    save_file({"a.weight": w, "a.weight_scale": torch.zeros(4, 4, dtype=torch.uint8),
               "b.weight": w.clone(), "b.weight_scale": torch.zeros(4, dtype=torch.uint8),
               "c.weight": torch.zeros(4, 128, dtype=torch.bfloat16)}, str(d / "m.safetensors"))
    (d / qc.MANIFEST).write_text(json.dumps({"spec": {"format": "mxfp8"}}))
    r = qc.QuantizedCheckpoint(d)
    assert r.format == "mxfp8" and "a.weight" in r and r.keys()[0] == "a.weight"
    codes, scales = r.fp8("a")
    assert codes.shape == (4, 128) and scales.shape == (4, 4)
    assert r.fp8("c") is None and r.fp8("nothing") is None
    with pytest.raises(ValueError, match="b.weight_scale"):
        r.fp8("b")
    with pytest.raises(KeyError):
        r.get("nothing")


@pytest.mark.parametrize("k", AWKWARD_K)
def test_oracle_mx_equals_the_reference_quantizer_at_awkward_k(k):
    """The oracle's MX law (codes and E8M0 scales) against the reference's own quantize_mx on
    the same seeded rows, K = 384 (one remainder tile) up to 13824."""
    q, s = omx.quantize_mx(awkward_rows(k))
    rec = GOLDEN["mx_awkward_k"][str(k)]
    assert tensor_digest(torch.from_numpy(q).view(torch.float8_e4m3fn)) == rec["codes"]
    assert tensor_digest(torch.from_numpy(s)) == rec["scales"]


def test_golden_tensor_digest_is_stable():
    """The fixture's digests are of the raw bytes: a plain sha256 of a known tensor."""
    t = torch.tensor([1.0, -2.0], dtype=torch.bfloat16)
    assert tensor_digest(t) == ["bfloat16", [2], hashlib.sha256(
        np.array([0x3F80, 0xC000], dtype=np.uint16).tobytes()).hexdigest()]


@pytest.mark.parametrize("model", ["flux", "qwen_image", "wan"])
def test_default_specs_are_the_reference_recipes(model):
    """difflet/quant/targets.py default_spec(model), as the reference wrote it: same targets,
    row-parallel and split patterns, so a directory written by `difflet compile --quant` for
    that model has the digest ours computes."""
    from difflet_amd.quant.spec import default_spec

    want = {k: v for k, v in GOLDEN["default_specs"][model].items() if k != "compute"}
    spec = default_spec(model)
    assert {k: v for k, v in spec.to_dict().items() if k != "compute"} == want
    rw = default_spec(model, format="fp8_rowwise")
    assert rw.split_linears == ()
    # the per-channel spec names the fused proj_out where the MXFP8 one names its halves
    fused = lambda pats: tuple(dict.fromkeys(p.replace("proj_out_(attn|mlp)", "proj_out")  # noqa: E731
                                             for p in pats))
    assert rw.targets == fused(spec.targets) and rw.row_parallel == fused(spec.row_parallel)
    with pytest.raises(ValueError, match="no fp8 target layers"):
        default_spec("ltx_2")


@pytest.mark.parametrize("fmt", ["mxfp8", "fp8_rowwise"])
def test_default_flux_spec_is_accepted_by_the_writer(toy, fmt):
    """Both formats' default FLUX spec pass the writer's checks on a FLUX directory: every
    target and row-parallel pattern names a weight the written directory holds."""
    from difflet_amd.quant.spec import default_spec

    spec = default_spec("flux", format=fmt)
    qc._validate(Path(toy), spec)
    shapes = qc._weight_shapes(Path(toy))
    names = qc._quantizable_prefixes(shapes, spec)
    single = [n for n in names if "single_transformer_blocks.0.proj_out" in n]
    want = ["proj_out_attn", "proj_out_mlp"] if fmt == "mxfp8" else ["proj_out"]
    assert sorted(n.rsplit(".", 1)[1] for n in single) == want
    assert all(spec.matches(n) for n in single)
