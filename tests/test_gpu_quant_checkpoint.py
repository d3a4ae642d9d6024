"""The quantized-checkpoint writer and loader on the GPU.

* mxfp8: the directory written through the HIP quantizer holds, key for key, the bytes the
  reference's own writer stored for the same toy and spec (every tensor's sha256, the index's
  shard map, the manifest), and the HIP quantizer equals the reference's quantize_mx at the
  awkward K values;
* fp8_rowwise: codes and scales equal the oracle's per-channel quantizer bit for bit, every other
  tensor is the source's;
* loading: a FLUX step built from the directory (codes and scales as stored, no quantization)
  gives exactly the output of the step that quantizes the same dense weights at load."""

from __future__ import annotations

import dataclasses
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from difflet_amd import kernels
from difflet_amd.dit.flux import FluxConfig, FluxDiT
from difflet_amd.dit.linear import DeviceLinear
from difflet_amd.quant import checkpoint as qc
from difflet_amd.quant.spec import FLUX_ALL_BLOCK_LINEARS, RocmQuantSpec
from oracle import fp8 as ofp8
from tests.golden.make_quant_checkpoint_golden import AWKWARD_K, awkward_rows
from tests.golden.quant_toy import tensor_digest, toy_tensors, write_toy_flux

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "quant_checkpoint_golden.json").read_text())
TOY_CFG = dict(hidden=512, heads=4, head_dim=128, n_double=1, n_single=1, txt_dim=896,
               pooled_dim=384)


def ours(label: str) -> RocmQuantSpec:
    body = dict(GOLDEN["specs"][label]["spec"], compute="rocm")
    return RocmQuantSpec.from_dict(body)


@pytest.fixture(scope="module")
def toy(tmp_path_factory):
    return write_toy_flux(tmp_path_factory.mktemp("toy"))


@pytest.mark.parametrize("label", sorted(GOLDEN["specs"]))
def test_mxfp8_directory_equals_the_reference_writer(gpu, toy, tmp_path, label):
    rec = GOLDEN["specs"][label]
    spec = ours(label)
    print(f"mxfp8 writer, spec {label}", flush=True)
    out = qc.quantized_dir(tmp_path / "cache", toy, spec)
    manifest = qc.write_quantized_dir(toy, out, spec, shard_bytes=GOLDEN["shard_bytes"], device=gpu)
    assert out.name == f"mxfp8-{rec['digest']}"
    want = rec["manifest"]
    for field in ("schema", "quantized_linears", "tensors", "bytes", "files"):
        assert manifest[field] == want[field], field
    assert manifest["source"]["fingerprint"] == want["source"]["fingerprint"]
    assert manifest["source"]["bytes"] == want["source"]["bytes"]
    assert {k: v for k, v in manifest["spec"].items() if k != "compute"} == \
        {k: v for k, v in want["spec"].items() if k != "compute"}
    index = json.loads((out / qc.INDEX_NAME).read_text())
    assert index["weight_map"] == rec["index_weight_map"]
    assert index["metadata"]["total_size"] == rec["index_total_size"]
    ckpt = qc.QuantizedCheckpoint(out)
    assert ckpt.keys() == sorted(rec["tensors"])
    bad = [k for k in ckpt.keys() if tensor_digest(ckpt.get(k)) != rec["tensors"][k]]
    assert not bad, f"tensors that differ from the reference writer's: {bad[:8]}"
    assert sorted(p.name for p in out.iterdir()
                  if not p.name.endswith((".safetensors", ".json"))) == rec["copied_files"]
    assert qc.check_quantized_dir(out, toy, spec) == qc.read_manifest(out)
    assert qc.ensure_quantized_dir(tmp_path / "cache", toy, spec, create=False) == out


@pytest.mark.parametrize("k", AWKWARD_K)
def test_hip_mx_quantizer_equals_the_reference_at_awkward_k(gpu, k):
    print(f"quantize_mxfp8 K={k}", flush=True)
    q, s = kernels.quantize_mxfp8(torch.from_numpy(awkward_rows(k)).to(gpu), swizzled=False)
    rec = GOLDEN["mx_awkward_k"][str(k)]
    assert tensor_digest(q.cpu()) == rec["codes"]
    assert tensor_digest(s.cpu()) == rec["scales"]


def test_fp8_rowwise_directory_matches_the_oracle(gpu, toy, tmp_path):
    targets = FLUX_ALL_BLOCK_LINEARS + (r"context_embedder",)
    spec = RocmQuantSpec(targets=targets, format="fp8_rowwise")
    out = tmp_path / "rw"
    print("fp8_rowwise writer", flush=True)
    manifest = qc.write_quantized_dir(toy, out, spec, shard_bytes=1 << 20, device=gpu)
    src = toy_tensors()
    ckpt = qc.QuantizedCheckpoint(out)
    assert ckpt.format == "fp8_rowwise"
    names = manifest["quantized_linears"]
    # 12 linears of the double block, 5 of the single block, the context embedder
    assert len(names) == 18 and manifest["tensors"]["quantized"] == 18
    assert manifest["tensors"]["total"] == len(src) + 18
    for name in names:
        codes, scales = ckpt.fp8(name)
        want_q, want_s = ofp8.quantize_rowwise(src[f"{name}.weight"].float().numpy())
        assert np.array_equal(codes.view(torch.uint8).numpy(), want_q), name
        assert np.array_equal(scales.numpy().view(np.uint32), want_s.view(np.uint32)), name
    for key, t in src.items():
        if key.endswith(".weight") and key[: -len(".weight")] in names:
            continue
        got = ckpt.get(key)
        assert got.dtype == t.dtype and torch.equal(got, t), key
    # the to_q edge rows: all-zero row -> zero codes; the 1e-30 row keeps a tiny scale
    codes, scales = ckpt.fp8("transformer_blocks.0.attn.to_q")
    assert not codes[0].view(torch.uint8).any() and scales[2] < 1e-30


def _inputs(gpu, img_hw=(16, 16), st=64, seed=3):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(1, img_hw[0] * img_hw[1], 64, generator=g)
    txt = torch.randn(1, st, 896, generator=g)
    pooled = torch.randn(1, 384, generator=g)
    return (lat.to(gpu), txt.to(gpu), pooled.to(gpu), torch.tensor([0.6], device=gpu),
            torch.tensor([3.5], device=gpu), img_hw)


def _same_linear(a: DeviceLinear, b: DeviceLinear, name: str) -> None:
    assert a.kind == b.kind, name
    assert torch.equal(a.w.view(torch.uint8) if a.kind != "bf16" else a.w,
                       b.w.view(torch.uint8) if b.kind != "bf16" else b.w), name
    if a.ws is not None:
        assert torch.equal(a.ws, b.ws), name
    assert torch.equal(a.bias, b.bias), name


def _linears(m: FluxDiT):
    for i, blk in enumerate(m.double):
        for n in ("qkv_img", "qkv_txt", "out_img", "out_txt", "ff1_img", "ff2_img", "ff1_txt", "ff2_txt"):
            yield f"double.{i}.{n}", getattr(blk, n)
    for i, blk in enumerate(m.single):
        yield f"single.{i}.w1", blk.w1
        yield f"single.{i}.w2", blk.w2


def test_flux_step_from_fp8_rowwise_directory_equals_quantize_at_load(gpu, toy, tmp_path):
    spec = RocmQuantSpec(targets=FLUX_ALL_BLOCK_LINEARS, format="fp8_rowwise")
    out = tmp_path / "rw"
    qc.write_quantized_dir(toy, out, spec, device=gpu)
    cfg = FluxConfig(**TOY_CFG)
    src = toy_tensors()
    print("FLUX toy step: fp8_rowwise directory vs quantize at load", flush=True)
    dense = FluxDiT(cfg, lambda n: src[n], kind="fp8", device=gpu)
    loaded = FluxDiT.from_quantized_dir(cfg, out, device=gpu)
    assert loaded.kind == "fp8"
    for (name, a), (_, b) in zip(_linears(dense), _linears(loaded)):
        _same_linear(a, b, name)
    y0 = dense(*_inputs(gpu))
    y1 = loaded(*_inputs(gpu))
    torch.cuda.synchronize()
    assert torch.isfinite(y0.float()).all()
    assert torch.equal(y0, y1)


def test_flux_step_from_mxfp8_directory_equals_quantize_at_load(gpu, toy, tmp_path):
    """The reference's FLUX MXFP8 spec: the double blocks' output projections stay bf16 and the
    single blocks' proj_out is stored as its two halves, fused back along K at load."""
    spec = ours("flux_mx")
    out = tmp_path / "mx"
    qc.write_quantized_dir(toy, out, spec, device=gpu)
    assert "single_transformer_blocks.0.proj_out_attn.weight" in qc.QuantizedCheckpoint(out)
    cfg = FluxConfig(**TOY_CFG)
    src = toy_tensors()
    print("FLUX toy step: mxfp8 directory vs quantize at load", flush=True)
    dense = FluxDiT(cfg, lambda n: src[n].to(gpu), kind="mx", device=gpu)
    for blk, pre in zip(dense.double, ["transformer_blocks.0"]):
        for attr, name in (("out_img", "attn.to_out.0"), ("out_txt", "attn.to_add_out")):
            setattr(blk, attr, DeviceLinear(src[f"{pre}.{name}.weight"].to(gpu),
                                            src[f"{pre}.{name}.bias"].to(gpu), "bf16"))
    loaded = FluxDiT.from_quantized_dir(cfg, out, device=gpu)
    assert loaded.kind == "mx"
    for (name, a), (_, b) in zip(_linears(dense), _linears(loaded)):
        _same_linear(a, b, name)
    y0 = dense(*_inputs(gpu))
    y1 = loaded(*_inputs(gpu))
    torch.cuda.synchronize()
    assert torch.isfinite(y0.float()).all()
    assert torch.equal(y0, y1)


def test_partly_quantized_group_is_refused(gpu, toy, tmp_path):
    spec = RocmQuantSpec(targets=(r"transformer_blocks\.\d+\.attn\.to_q",), format="fp8_rowwise")
    out = tmp_path / "part"
    qc.write_quantized_dir(toy, out, spec, device=gpu)
    with pytest.raises(ValueError, match="quantized all together or not at all"):
        FluxDiT.from_quantized_dir(FluxConfig(**TOY_CFG), out, device=gpu)


def test_fp8_twins_load_from_the_directory(gpu, toy, tmp_path):
    """The quantized-linear API: quantize_module_ leaves empty twins, load_fp8_linears_ fills them
    from the directory, and each twin's output equals the twin quantized from the dense weight."""
    import torch.nn as nn

    from difflet_amd.quant.linear import prepare_fp8_kernels_, quantize_module_

    spec = RocmQuantSpec(targets=(r"transformer_blocks\.\d+\.ff\.net\.(0\.proj|2)",),
                         format="fp8_rowwise")
    out = tmp_path / "twins"
    qc.write_quantized_dir(toy, out, spec, device=gpu)
    src = toy_tensors()

    def module():
        m = nn.Module()
        ff = nn.ModuleDict({"0": nn.Module(), "2": nn.Linear(2048, 512)})
        ff["0"].proj = nn.Linear(512, 2048)
        m.transformer_blocks = nn.ModuleList([nn.Module()])
        m.transformer_blocks[0].ff = nn.Module()
        m.transformer_blocks[0].ff.net = ff
        for n, p in (("0.proj", ff["0"].proj), ("2", ff["2"])):
            p.weight.data = src[f"transformer_blocks.0.ff.net.{n}.weight"].float()
            p.bias.data = src[f"transformer_blocks.0.ff.net.{n}.bias"].float()
        return m.to(gpu)

    a, b = module(), module()
    quantize_module_(a, spec, from_dense=True)
    quantize_module_(b, spec)
    filled = qc.load_fp8_linears_(b, out)
    assert sorted(filled) == ["transformer_blocks.0.ff.net.0.proj", "transformer_blocks.0.ff.net.2"]
    prepare_fp8_kernels_(a)
    prepare_fp8_kernels_(b)
    x = torch.randn(64, 512, device=gpu, dtype=torch.bfloat16)
    for m in (a, b):
        m.y = m.transformer_blocks[0].ff.net["2"](m.transformer_blocks[0].ff.net["0"].proj(x))
    assert torch.equal(a.y, b.y)
    mx_spec = dataclasses.replace(spec, format="mxfp8")
    c = module()
    quantize_module_(c, mx_spec)
    with pytest.raises(ValueError, match="holds fp8_rowwise"):
        qc.load_fp8_linears_(c, out)


def test_qwen_step_from_mxfp8_directory_equals_quantize_at_load(gpu, tmp_path):
    """Qwen-Image with the reference's default MXFP8 targets, from a single-file source (no
    index): the step loaded from the directory equals the step quantizing at load."""
    from safetensors.torch import save_file

    from difflet_amd.dit.qwen import QwenConfig, QwenImageDiT, qwen_param_shapes
    from difflet_amd.quant.spec import QWEN_IMAGE_TARGETS

    cfg = QwenConfig(hidden=512, heads=4, mlp=2048, n_blocks=2, txt_dim=896)
    g = torch.Generator().manual_seed(5)
    src = {}
    for name, shape in sorted(qwen_param_shapes(cfg).items()):
        t = torch.randn(shape, generator=g) * (0.1 if len(shape) == 1 else 0.02)
        src[name] = (t + 1.0 if "norm" in name and len(shape) == 1 else t).to(torch.bfloat16)
    d = tmp_path / "qwen" / "transformer"
    d.mkdir(parents=True)
    save_file(src, str(d / "diffusion_pytorch_model.safetensors"), metadata={"format": "pt"})
    spec = RocmQuantSpec(targets=QWEN_IMAGE_TARGETS)
    out = tmp_path / "mx"
    manifest = qc.write_quantized_dir(d, out, spec, device=gpu)
    assert manifest["tensors"]["quantized"] == 2 * 10 and len(manifest["files"]) == 1
    print("Qwen toy step: mxfp8 directory vs quantize at load", flush=True)
    dense = QwenImageDiT(cfg, lambda n: src[n], kind="mx", device=gpu)
    loaded = QwenImageDiT.from_quantized_dir(cfg, out, device=gpu)
    assert loaded.kind == "mx"
    for blk_a, blk_b in zip(dense.blocks, loaded.blocks):
        for n in ("qkv_img", "qkv_txt", "out_img", "out_txt", "ff1_img", "ff2_img", "ff1_txt", "ff2_txt"):
            _same_linear(getattr(blk_a, n), getattr(blk_b, n), n)
    g = torch.Generator().manual_seed(6)
    lat = torch.randn(1, 16 * 16, 64, generator=g).to(gpu)
    txt = torch.randn(1, 40, 896, generator=g).to(gpu)
    t = torch.tensor([0.4], device=gpu)
    y0 = dense(lat, txt, t, (16, 16))
    y1 = loaded(lat, txt, t, (16, 16))
    torch.cuda.synchronize()
    assert torch.isfinite(y0.float()).all()
    assert torch.equal(y0, y1)
