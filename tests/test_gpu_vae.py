"""FLUX's VAE decoder on the HIP path against the fp32 oracle (oracle/vae.py): the kernels
(GroupNorm, im2col, row softmax) alone, small decoders in fp32 (rel L2 <= 1e-4) and bf16 against
the oracle with the device's rounding points (<= 2e-2), a real-width resnet and the mid-block
attention at FLUX's 512 channels, and the full 128 x 128 -> 1024 x 1024 decode through
properties."""

import dataclasses

import pytest
import torch
import torch.nn.functional as F

from difflet_amd import kernels
from difflet_amd.vae import decoder as dvae
from oracle import vae as ovae

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _cfg(shape: ovae.VaeShape) -> dvae.VaeConfig:
    return dvae.VaeConfig(latent_channels=shape.latent_channels, out_channels=shape.out_channels,
                          block_out_channels=tuple(shape.block_out_channels),
                          layers_per_block=shape.layers_per_block, norm_num_groups=shape.groups)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("c,pix", [(128, 1000), (512, 4096), (256, 37), (16, 300)])
def test_group_norm_matches_torch(gpu, dtype, c, pix):
    g = torch.Generator().manual_seed(c + pix)
    groups = 32 if c % 32 == 0 else 8
    x = (torch.randn(2, pix, c, generator=g) * 2 + 3).to(dtype)
    w, b = torch.randn(c, generator=g), torch.randn(c, generator=g)
    ref = F.group_norm(x.float().permute(0, 2, 1), groups, w, b, 1e-6).permute(0, 2, 1)
    out = kernels.group_norm(x.to(gpu), groups, w.to(gpu), b.to(gpu), 1e-6)
    tol = 2e-6 if dtype == torch.float32 else 5e-3
    assert out.dtype == dtype and rel_l2(out, ref) < tol
    out = kernels.group_norm(x.to(gpu), groups, w.to(gpu), b.to(gpu), 1e-6, silu=True)
    assert rel_l2(out, F.silu(ref)) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("h,w,c,up", [(5, 7, 16, False), (5, 7, 16, True), (33, 20, 64, True),
                                      (1, 1, 8, False)])
def test_im2col_rows_are_exact(gpu, dtype, h, w, c, up):
    if dtype == torch.float32 and c % 4:
        pytest.skip("fp32 needs C % 4")
    g = torch.Generator().manual_seed(h * w + c)
    x = torch.randn(h, w, c, generator=g).to(dtype)
    xi = x.permute(2, 0, 1)[None]
    if up:
        xi = F.interpolate(xi.float(), scale_factor=2.0, mode="nearest").to(dtype)
    ho, wo = xi.shape[2:]
    hwc = F.pad(xi[0].permute(1, 2, 0), (0, 0, 1, 1, 1, 1))
    rows = torch.stack([hwc[ky:ky + ho, kx:kx + wo] for ky in range(3) for kx in range(3)], 2)
    kp = -(-9 * c // 64) * 64 + 64
    ref = F.pad(rows.reshape(ho * wo, 9 * c), (0, kp - 9 * c))
    out = kernels.im2col3x3(x.to(gpu), upsample=up, kpad=kp)
    assert torch.equal(out.cpu(), ref)
    if ho * wo > 8:  # a chunk of output pixels, as the decoder's chunked convolutions take
        part = kernels.im2col3x3(x.to(gpu), upsample=up, kpad=kp, row0=3, rows=5)
        assert torch.equal(part.cpu(), ref[3:8])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cols,ld", [(1030, 1030), (1024, 1024), (6241, 6244), (15, 16)])
def test_softmax_rows(gpu, dtype, cols, ld):
    """Rows in 16-byte runs (ld a multiple of 4) and one element at a time (1030), a ragged tail
    (6241, 15), and a row maximum that moves late (a ramp), against torch.softmax."""
    g = torch.Generator().manual_seed(5 + cols)
    s = torch.randn(300, ld, generator=g) * 20
    s[:, : cols // 2] -= 40.0  # the running maximum jumps halfway along each row
    out = torch.empty(300, ld, dtype=dtype, device=gpu)[:, :cols]
    kernels.softmax_rows(s.to(gpu)[:, :cols], 0.044, dtype=dtype, out=out)
    ref = torch.softmax(s[:, :cols] * 0.044, dim=-1)
    assert rel_l2(out, ref) < (2e-6 if dtype == torch.float32 else 4e-3)


SMALL = ovae.VaeShape(latent_channels=16, block_out_channels=(32, 32, 64, 64), layers_per_block=1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hw", [(8, 8), (6, 10)])
def test_small_decoder_matches_oracle(gpu, dtype, hw, parity):
    """Four up blocks of two resnets (one with a 1x1 shortcut, 64 -> 32 channels), three
    upsamplings, the mid-block attention over 64 or 60 latent pixels (60: the P V GEMM's K
    padded). bf16 within 2e-2: this random-weight decoder stored in bf16 moves 1.25e-2 when the
    oracle itself only sums its convolutions in fp64 instead of fp32 (the rounding flips of
    one layer change the next layer's), so 1e-2 sits below the oracle's own noise."""
    print(f"vae small {dtype} {hw}", flush=True)
    w = ovae.weights(SMALL, 8, None if dtype == torch.float32 else dtype)
    dec = dvae.VaeDecoder(_cfg(SMALL), lambda n: w[n], dtype=dtype, device=gpu)
    z = torch.randn(1, 16, *hw, generator=torch.Generator().manual_seed(9))
    store = None if dtype == torch.float32 else dtype
    ref = ovae.decode(w, SMALL, z, store=store)
    out = dec.decode(z.to(gpu))
    torch.cuda.synchronize()
    assert out.dtype == dtype and tuple(out.shape) == tuple(ref.shape)
    e = rel_l2(out, ref)
    print(f"  rel L2 {e:.3e}", flush=True)
    bound = 1e-4 if dtype == torch.float32 else 2e-2
    parity(f"small FLUX VAE decode {str(dtype)[6:]}, rel L2 vs oracle at the device's rounding "
           "points", e, bound)
    assert e < bound


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_flux_width_resnet_and_attention_match_oracle(gpu, dtype):
    """FLUX's mid block pieces at 512 channels on a 32 x 32 latent (1024 pixels): a resnet,
    the attention, and the 512 -> 256 resnet with its shortcut at 64 x 64."""
    w = ovae.weights(ovae.FLUX_VAE, 10, None if dtype == torch.float32 else dtype)
    dec = dvae.VaeDecoder(dvae.FLUX_VAE, lambda n: w[n], dtype=dtype, device=gpu)
    store = None if dtype == torch.float32 else dtype
    r = (lambda t: t) if store is None else (lambda t: t.to(store).float())
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    g = torch.Generator().manual_seed(11)
    x = r(torch.randn(1, 512, 32, 32, generator=g))
    hwc = x[0].permute(1, 2, 0).reshape(1024, 512).to(gpu, dtype).contiguous()
    pre = "decoder.mid_block.resnets.0"
    ref = ovae.resnet(w, pre, x, ovae.FLUX_VAE, r)
    out = dec._resnet(hwc, (32, 32), pre)
    assert rel_l2(out.reshape(32, 32, 512).permute(2, 0, 1), ref[0]) < tol
    pre = "decoder.mid_block.attentions.0"
    ref = ovae.attention(w, pre, x, ovae.FLUX_VAE, r)
    out = dec._attention(hwc)
    assert rel_l2(out.reshape(32, 32, 512).permute(2, 0, 1), ref[0]) < tol
    x = r(torch.randn(1, 512, 64, 64, generator=g))
    pre = "decoder.up_blocks.2.resnets.0"
    ref = ovae.resnet(w, pre, x, ovae.FLUX_VAE, r)
    out = dec._resnet(x[0].permute(1, 2, 0).reshape(4096, 512).to(gpu, dtype).contiguous(), (64, 64), pre)
    assert rel_l2(out.reshape(64, 64, 256).permute(2, 0, 1), ref[0]) < tol


def test_flux_vae_full_decode_bf16_and_fp32(gpu):
    """FLUX.1's decoder (128 x 128 x 16 latent -> 1024 x 1024 RGB) with random weights: both
    dtypes finite and bit-identical on a rerun, bf16 within 5e-2 of fp32."""
    z = torch.randn(1, 16, 128, 128, generator=torch.Generator().manual_seed(12)).to(gpu)
    outs = {}
    for dt in (torch.float32, torch.bfloat16):
        print(f"flux vae full decode {dt}", flush=True)
        dec = dvae.VaeDecoder(dvae.FLUX_VAE, dvae.random_param_source(dvae.FLUX_VAE, 3, gpu),
                              dtype=dt, device=gpu)
        a, b = dec.decode(z), dec.decode(z)
        torch.cuda.synchronize()
        assert tuple(a.shape) == (1, 3, 1024, 1024)
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a, b)
        outs[dt] = a.float().cpu()
        del dec, a, b
        torch.cuda.empty_cache()
    e = rel_l2(outs[torch.bfloat16], outs[torch.float32])
    print(f"  bf16 vs fp32 rel L2 {e:.3e}", flush=True)
    assert e < 5e-2


@pytest.mark.parametrize("m,n,k", [(1000, 1003, 384), (6240, 6240, 384), (300, 4096, 512)])
def test_bf16_gemm_with_fp32_output(gpu, m, n, k):
    """The mid-block attention's scores: bf16 q k^T with the fp32 accumulators stored as they
    are (the products exact, sums in fp32), keys padded to a multiple of 4."""
    print(f"bf16 gemm fp32 out {m} x {n} x {k}", flush=True)
    g = torch.Generator().manual_seed(m + n)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = torch.randn(n, k, generator=g).to(torch.bfloat16)
    s = kernels.gemm_bf16_f32out(a.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    assert s.dtype == torch.float32 and tuple(s.shape) == (m, n)
    ref = a.double() @ w.double().t()
    assert rel_l2(s, ref) < 1e-6
