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


def test_wan_block_matches_fp32_oracle(gpu):
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
    assert e < 1e-2


def test_wan_reduced_depth_step_matches_fp32_oracle(gpu):
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
    assert out.shape == (1, 16, 3, 12, 10)
    assert e < 1e-2
