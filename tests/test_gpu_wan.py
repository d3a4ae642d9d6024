"""Wan blocks and a reduced-depth Wan step on the HIP path against the fp32 oracle (bf16,
rel L2 <= 1e-2)."""

import torch
import pytest

from difflet_amd import kernels
from difflet_amd.dit.wan import WanConfig, WanDiT
from oracle import wan as owan

pytestmark = pytest.mark.gpu

SEED = 777


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _source(shape, n_blocks, seed=SEED):
    w = dict(owan.embed_weights(shape, seed))
    for i in range(n_blocks):
        for k, v in owan.block_weights(shape, seed, i).items():
            w[f"blocks.{i}.{k}"] = v
    return w


def test_wan_block_matches_fp32_oracle(gpu, parity):
    """One block at Wan-14B width (5120, 40 heads, FFN 13824) on a 3 x 10 x 12 patch grid
    (360 video tokens) with 96 text tokens."""
    print("wan block", flush=True)
    shape = owan.WanShape(n_blocks=1)
    w = _source(shape, 1)
    dit = WanDiT(WanConfig(n_blocks=1), lambda n: w[n], device=gpu)
    grid, st = (3, 10, 12), 96
    s = grid[0] * grid[1] * grid[2]
    g = torch.Generator().manual_seed(SEED)
    hidden = torch.randn(1, s, shape.hidden, generator=g).bfloat16().float()
    text = torch.randn(1, st, shape.hidden, generator=g).bfloat16().float()
    tproj = (torch.randn(1, 6, shape.hidden, generator=g) * 0.5).bfloat16().float()
    cos, sin = owan.rope_tables(grid, shape)
    bw = {k[len("blocks.0."):]: v for k, v in w.items() if k.startswith("blocks.0.")}
    ref = owan.block(bw, hidden, text, tproj, cos, sin, shape)
    bufs = dit._buffers(s, st)
    bufs["h"].copy_(hidden[0].to(gpu, torch.bfloat16))
    bufs["txt"].copy_(text[0].to(gpu, torch.bfloat16))
    mods = dit.sst[0] + tproj[0].to(gpu)
    gates = mods[2::3].to(torch.bfloat16).contiguous()
    gcos, gsin = dit.rope_tables(grid)
    dit.block(0, bufs, mods, gates, gcos, gsin)
    torch.cuda.synchronize()
    e = rel_l2(bufs["h"], ref[0])
    print(f"block rel L2 {e:.3e}", flush=True)
    parity("block at Wan-14B width, rel L2 vs fp32 oracle", e, 1e-2)
    assert e < 1e-2


def test_wan_reduced_depth_step_matches_fp32_oracle(gpu, parity):
    """Patch embedding, time / text conditioning, 2 blocks, norm_out, proj_out and unpatchify on
    latents [1, 16, 3, 12, 10] (3 x 6 x 5 patches) with 48 text tokens of 4096."""
    print("wan reduced step", flush=True)
    shape = owan.WanShape(n_blocks=2)
    w = _source(shape, 2)
    inp = owan.synthetic_inputs(shape, SEED, (3, 12, 10), 48)
    lat, txt = inp["latents"].bfloat16().float(), inp["text"].bfloat16().float()
    ref = owan.forward(shape, SEED, lat, inp["timestep"], txt,
                       weights=(owan.embed_weights(shape, SEED),
                                [owan.block_weights(shape, SEED, i) for i in range(2)]),
                       model_dtype=torch.bfloat16)
    dit = WanDiT(WanConfig(n_blocks=2), lambda n: w[n], device=gpu)
    out = dit.forward(lat.to(gpu), inp["timestep"].to(gpu), txt.to(gpu))
    torch.cuda.synchronize()
    e = rel_l2(out, ref)
    print(f"step rel L2 {e:.3e}", flush=True)
    parity("2-block step, rel L2 vs fp32 oracle", e, 1e-2)
    assert out.shape == (1, 16, 3, 12, 10)
    assert e < 1e-2


def test_wan_block_mx_matches_the_oracle_of_the_same_law(gpu, parity):
    """The reference's MXFP8 Wan targets (cross-attention q/k/v, both FFN linears) on the MX
    GEMM, against the oracle block with the MX law on the same linears and the device's bf16
    rounding points (rel L2 <= 3e-2), at width 1024 (8 heads), FFN 2816, a 2 x 8 x 8 grid and
    64 text tokens; the device's error against the unquantized block equals the oracle's own
    within 10 %."""
    print("wan block, mx", flush=True)
    kw = dict(hidden=1024, heads=8, ffn=2816, n_blocks=1)
    shape = owan.WanShape(**kw)
    w = _source(shape, 1)
    dit = WanDiT(WanConfig(**kw), lambda n: w[n], device=gpu, kind="mx")
    assert [getattr(dit.blocks[0], n).kind for n in ("qkv", "out1", "q2", "kv2", "out2", "ffn_in",
                                                      "ffn_out")] == ["bf16", "bf16", "mx", "mx", "bf16", "mx", "mx"]
    grid, st = (2, 8, 8), 64
    s = grid[0] * grid[1] * grid[2]
    g = torch.Generator().manual_seed(SEED + 1)
    hidden = torch.randn(1, s, shape.hidden, generator=g).bfloat16().float()
    text = torch.randn(1, st, shape.hidden, generator=g).bfloat16().float()
    tproj = (torch.randn(1, 6, shape.hidden, generator=g) * 0.5).bfloat16().float()
    cos, sin = owan.rope_tables(grid, shape)
    bw = {k[len("blocks.0."):]: v.float() for k, v in w.items() if k.startswith("blocks.0.")}
    ref = owan.block(bw, hidden, text, tproj, cos, sin, shape, quant="mx", act_dtype=torch.bfloat16,
                     store=torch.bfloat16)
    ref_bf16 = owan.block(bw, hidden, text, tproj, cos, sin, shape)
    bufs = dit._buffers(s, st)
    bufs["h"].copy_(hidden[0].to(gpu, torch.bfloat16))
    bufs["txt"].copy_(text[0].to(gpu, torch.bfloat16))
    mods = dit.sst[0] + tproj[0].to(gpu)
    gates = mods[2::3].to(torch.bfloat16).contiguous()
    gcos, gsin = dit.rope_tables(grid)
    dit.block(0, bufs, mods, gates, gcos, gsin)
    torch.cuda.synchronize()
    e = rel_l2(bufs["h"], ref[0])
    fmt_dev, fmt_ref = rel_l2(bufs["h"], ref_bf16[0]), rel_l2(ref, ref_bf16)
    print(f"mx block rel L2 vs the MX oracle {e:.3e}; format error device {fmt_dev:.3e}, "
          f"oracle {fmt_ref:.3e}", flush=True)
    parity("mx block, rel L2 vs same-law oracle", e, 3e-2)
    parity(f"mx block, format error vs fp32 (oracle's {fmt_ref:.3e})", fmt_dev, 6e-2)
    assert e < 3e-2
    assert abs(fmt_dev - fmt_ref) <= 0.1 * fmt_ref


def test_wan_step_from_mxfp8_directory_equals_quantize_at_load(gpu, tmp_path):
    """A Wan checkpoint under diffusers' names (ffn.net.0.proj / ffn.net.2), quantized with the
    reference's Wan targets: the step built from the directory equals the step that quantizes
    the same weights at load."""
    from safetensors.torch import save_file

    from difflet_amd.dit.wan import checkpoint_key, wan_param_shapes
    from difflet_amd.quant import checkpoint as qc
    from difflet_amd.quant.spec import WAN_TARGETS, RocmQuantSpec

    cfg = WanConfig(hidden=512, heads=4, ffn=1536, n_blocks=2, text_dim=256)
    g = torch.Generator().manual_seed(9)
    src = {n: (torch.randn(shp, generator=g) * 0.02).to(torch.bfloat16)
           for n, shp in sorted(wan_param_shapes(cfg).items())}
    d = tmp_path / "wan" / "transformer"
    d.mkdir(parents=True)
    save_file({checkpoint_key(n): t for n, t in src.items()},
              str(d / "diffusion_pytorch_model.safetensors"), metadata={"format": "pt"})
    out = tmp_path / "mx"
    manifest = qc.write_quantized_dir(d, out, RocmQuantSpec(targets=WAN_TARGETS), device=gpu)
    assert manifest["tensors"]["quantized"] == 2 * 5
    print("Wan toy step: mxfp8 directory vs quantize at load", flush=True)
    dense = WanDiT(cfg, lambda n: src[n], device=gpu, kind="mx")
    loaded = WanDiT.from_quantized_dir(cfg, out, device=gpu)
    assert loaded.kind == "mx"
    g = torch.Generator().manual_seed(10)
    lat = torch.randn(1, 16, 2, 8, 8, generator=g).to(gpu)
    txt = torch.randn(1, 32, 256, generator=g).to(gpu)
    t = torch.tensor([700.0], device=gpu)
    y0 = dense(lat, t, txt)
    y1 = loaded(lat, t, txt)
    torch.cuda.synchronize()
    assert torch.isfinite(y0.float()).all()
    assert torch.equal(y0, y1)
