"""Wan's 3D causal VAE decoder on the HIP path: its kernels against torch statements of their
contracts (bit-exact gathers, fp32-law norms), decoders against the fp32 oracle
(oracle/wan_vae.py: fp32 <= 1e-4, bf16 <= 2e-2 against the oracle with the device's rounding
points: a random-weight decoder stored in bf16 moves 1.5-6.8e-3 when the oracle only sums its
convolutions in fp64, and 1.3-1.5e-2 from its fp32 form), Wan's real widths on a small latent, and the full 21-frame 480 x 832 decode through
properties (finite, bit-identical rerun, causal frame by frame, the first frame alone)."""

import pytest
import torch
import torch.nn.functional as F

from difflet_amd import _lib, kernels
from difflet_amd.vae import wan as dwan
from oracle import wan_vae as ow
from tests.test_wan_vae_host import _cfg, _im2col_causal

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


CASES = [  # (kt, ks, up, fpb, cache, frames, h, w, c)
    (3, 3, False, 1, True, 2, 5, 7, 16),
    (3, 3, False, 1, False, 1, 4, 6, 96),
    (3, 1, False, 1, True, 3, 3, 5, 64),    # a time convolution
    (1, 3, True, 1, False, 1, 5, 7, 16),     # the resampler's conv after chunk 0
    (1, 3, True, 2, False, 4, 3, 4, 8),      # ... reading the interleaved time-conv output
    (1, 1, False, 1, False, 3, 2, 9, 24),    # post_quant_conv / a padded 1x1
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", CASES)
def test_im2col_causal_rows_are_exact(gpu, dtype, case):
    kt, ks, up, fpb, with_cache, frames, h, w, c = case
    g = torch.Generator().manual_seed(sum(case[5:]))
    pix = h * w
    if fpb == 2:  # [frames / 2][pix][2C] holding frames 2t (channels [0, C)) and 2t + 1
        x = torch.randn(frames // 2, pix, 2 * c, generator=g).to(dtype)
        kw = dict(frames_per_block=2, frame_stride=pix * 2 * c, sub_stride=c, pixel_stride=2 * c)
    else:
        x = torch.randn(frames, pix, c, generator=g).to(dtype)
        kw = {}
    cache = torch.randn(2, pix, c, generator=g).to(dtype) if with_cache else None
    k = kt * ks * ks * c
    kpad = -(-k // 64) * 64 + 64
    po = pix * (4 if up else 1)
    rows = frames * po
    ref = _im2col_causal(x, (h, w), c, kt=kt, ks=ks, kpad=kpad, upsample=up, cache=cache,
                         row0=0, rows=rows, **kw)
    out = kernels.im2col_causal(x.to(gpu), (h, w), c, kt=kt, ks=ks, kpad=kpad, upsample=up,
                                cache=None if cache is None else cache.to(gpu), row0=0,
                                rows=rows, **kw)
    assert torch.equal(out.cpu(), ref)
    if rows > 9:  # a row range, as the decoder's chunked convolutions take
        part = kernels.im2col_causal(x.to(gpu), (h, w), c, kt=kt, ks=ks, kpad=kpad, upsample=up,
                                     cache=None if cache is None else cache.to(gpu), row0=4,
                                     rows=5, **kw)
        assert torch.equal(part.cpu(), ref[4:9])


def test_im2col_causal_refuses_an_overrun(gpu):
    x = torch.zeros(2, 12, 16, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="overrun"):
        kernels.im2col_causal(x, (3, 4), 16, kt=3, ks=3, kpad=448, row0=0, rows=3 * 12)


# (kt, ks, up, fpb, lead, frames, h, w, cin, cout, residual): every tile shape (cout <= 32, 64,
# 96 in one channel tile of 512 pixels; wider in 256 x 128 or 256 x 192 tiles, up to 4 across),
# taps that straddle the 64-column stages (C = 96, 8, 16), pixel counts that end mid-tile
CONV_CASES = [
    (3, 3, False, 1, 2, 2, 5, 7, 16, 4, False),      # conv_out-like, a 2-frame cache
    (3, 3, False, 1, 0, 1, 4, 6, 96, 96, True),      # the first chunk: zero padding in front
    (3, 3, False, 1, 2, 4, 12, 20, 96, 96, True),    # the full-resolution stage's widths
    (3, 3, False, 1, 2, 1, 9, 13, 8, 64, False),
    (3, 3, False, 1, 2, 2, 12, 20, 192, 192, False),
    (3, 3, False, 1, 2, 1, 6, 10, 384, 384, True),
    (3, 3, False, 1, 2, 3, 6, 10, 16, 384, False),   # conv_in
    (3, 1, False, 1, 2, 1, 6, 10, 384, 768, False),  # a time convolution
    (1, 3, True, 1, 0, 1, 6, 10, 384, 192, False),   # the resampler's conv after chunk 0
    (1, 3, True, 2, 0, 4, 3, 4, 8, 32, False),       # ... reading the interleaved time-conv output
    (1, 3, True, 2, 0, 2, 12, 20, 192, 96, False),
    (1, 1, False, 1, 0, 3, 2, 9, 24, 24, False),     # post_quant_conv-like 1x1
    (1, 3, False, 1, 0, 1, 20, 24, 128, 128, True),  # FLUX's 2D decoder: 256 x 128 tiles
    (1, 3, True, 1, 0, 1, 10, 12, 512, 256, False),  # ... two of them across
    (1, 3, False, 1, 0, 1, 8, 9, 512, 512, True),    # ... three 256 x 192 tiles
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_causal_equals_the_im2col_gemm(gpu, case, dtype):
    """The implicit GEMM against im2col rows times the weight on the whole-tile GEMM kernel of
    its dtype (bf16 matrix cores; fp32: the fp32 GEMM): the same products in the same order, so
    bit-identical (and the residual may be the output); both within output rounding of the
    fp32 convolution of the rows."""
    kt, ks, up, fpb, lead, frames, h, w, cin, cout, with_res = case
    print(f"conv_causal {case} {dtype}", flush=True)
    g = torch.Generator().manual_seed(cin * 7 + cout + frames)
    pix = h * w
    dt = dtype
    if fpb == 2:
        x = torch.randn(frames // 2, pix, 2 * cin, generator=g).to(dt)
        kw = dict(frames_per_block=2, frame_stride=pix * 2 * cin, sub_stride=cin,
                  pixel_stride=2 * cin)
        cache = None
    else:
        x = torch.randn(lead + frames, pix, cin, generator=g).to(dt)
        kw = {}
        cache = x[:2] if lead else None
    k = kt * ks * ks * cin
    kpad = -(-k // 64) * 64
    n = -(-cout // 4) * 4
    wt = torch.zeros(n, kpad)
    wt[:cout, :k] = torch.randn(cout, k, generator=g) * k ** -0.5
    wt = wt.to(dt)
    bias = (torch.randn(n, generator=g) * 0.1).to(dt)
    rows = frames * pix * (4 if up else 1)
    res = (torch.randn(rows, n, generator=g)).to(dt) if with_res else None
    xg, wg, bg = x.to(gpu), wt.to(gpu), bias.to(gpu)
    out = kernels.conv_causal(xg, (h, w), cin, frames, wg, bg, kt=kt, ks=ks, upsample=up,
                              lead_frames=lead, residual=None if res is None else res.to(gpu),
                              split=False, **kw)
    src = xg[lead:] if fpb == 1 else xg
    cols = kernels.im2col_causal(src.contiguous(), (h, w), cin, kt=kt, ks=ks, kpad=kpad,
                                 upsample=up, cache=None if cache is None else cache.to(gpu),
                                 rows=rows, **kw)
    ref = torch.empty(rows, n, dtype=dt, device=gpu)
    if dt == torch.float32:
        kernels.gemm_f32(cols, wg, bg, residual=None if res is None else res.to(gpu), out=ref)
    elif res is None:
        kernels.gemm_grouped([kernels.Problem(cols, wg, ref, bg)], kind="bf16")
    else:
        ones = torch.ones(1, n, dtype=dt, device=gpu)
        kernels.gemm_grouped([kernels.Problem(cols, wg, ref, bg, gate=ones,
                                              residual=res.to(gpu))],
                             kind="bf16", epilogue=_lib.EPI_GATE_RESIDUAL)
    torch.cuda.synchronize()
    bits = torch.int16 if dt == torch.bfloat16 else torch.int32
    assert torch.equal(out.view(bits), ref.view(bits))
    f32 = cols.float().cpu() @ wt.float().t() + bias.float()
    if res is not None:
        f32 = f32 + res.float()
        inplace = res.to(gpu)
        kernels.conv_causal(xg, (h, w), cin, frames, wg, bg, kt=kt, ks=ks, upsample=up,
                            lead_frames=lead, residual=inplace, out=inplace, split=False, **kw)
        torch.cuda.synchronize()
        assert torch.equal(inplace.view(bits), ref.view(bits))
    assert rel_l2(out, f32) < (4e-3 if dt == torch.bfloat16 else 1e-5)


@pytest.mark.parametrize("case", [
    (3, 3, 1, 60, 104, 384, 384, True),   # the latent-resolution resnet convolution: 50 tiles
    (3, 1, 1, 60, 104, 384, 768, False),  # the time convolution there (K = 1152)
    (3, 3, 2, 9, 13, 96, 96, True),       # 3 tiles of 512 x 96
    (3, 3, 1, 5, 7, 96, 4, False),        # 41 stages, 1 tile of 512 x 32: cut in 5
])
def test_conv_causal_split_k_matches_whole_tiles(gpu, case):
    """Convolutions under half a wave of tiles cut their K stages into ranges (up to 8, at
    least 8 stages each) whose fp32 partial sums a second kernel adds in order with the bias
    and the residual: within fp32 summation order of whole tiles (bf16 outputs at most one
    rounding step apart where no sum cancels), bit-identical on a rerun; whole tiles without a
    workspace."""
    kt, ks, frames, h, w, cin, cout, with_res = case
    print(f"conv_causal split {case}", flush=True)
    g = torch.Generator().manual_seed(cin + cout + h)
    bf, pix = torch.bfloat16, h * w
    x = torch.randn(2 + frames, pix, cin, generator=g).to(bf).to(gpu)
    k = kt * ks * ks * cin
    kpad = -(-k // 64) * 64
    n = -(-cout // 4) * 4
    wt = torch.zeros(n, kpad)
    wt[:cout, :k] = torch.randn(cout, k, generator=g) * k ** -0.5
    wt = wt.to(bf).to(gpu)
    bias = (torch.randn(n, generator=g) * 0.1).to(bf).to(gpu)
    rows = frames * pix
    res = torch.randn(rows, n, generator=g).to(bf).to(gpu) if with_res else None
    assert kernels.lib().difflet_rocm_conv_causal_workspace_bytes(rows, n, kpad) > 0
    run = lambda split: kernels.conv_causal(x, (h, w), cin, frames, wt, bias, kt=kt, ks=ks,
                                            lead_frames=2, residual=res, split=split)
    a, b, whole = run(True), run(True), run(False)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    d = (a.float() - whole.float()).abs()
    assert (d <= whole.float().abs() * 2 ** -7 + 1e-3).all() and rel_l2(a, whole) < 2e-3
    cols = kernels.im2col_causal(x[2:].contiguous(), (h, w), cin, kt=kt, ks=ks, kpad=kpad,
                                 cache=x[:2].contiguous())
    f32 = cols.float() @ wt.float().t() + bias.float() + (0 if res is None else res.float())
    assert rel_l2(a, f32.cpu()) < 4e-3


def test_conv_causal_full_resolution_stage(gpu):
    """A 96-channel 3x3x3 convolution of the full-resolution stage (4 frames of 480 x 832 and
    the 2-frame cache, 1.6 M output pixels, 3120 tiles) bit-identical to the im2col GEMM."""
    print("conv_causal 480x832x4 C=96", flush=True)
    g = torch.Generator(device=gpu).manual_seed(5)
    bf, h, w, c = torch.bfloat16, 480, 832, 96
    x = torch.randn(6, h * w, c, generator=g, device=gpu).to(bf)
    wt = torch.zeros(c, 2624, device=gpu)
    wt[:, :2592] = torch.randn(c, 2592, generator=g, device=gpu) * 2592 ** -0.5
    wt = wt.to(bf)
    bias = (torch.randn(c, generator=g, device=gpu) * 0.1).to(bf)
    out = kernels.conv_causal(x, (h, w), c, 4, wt, bias, kt=3, ks=3, lead_frames=2, split=False)
    ref = torch.empty_like(out)
    po = h * w
    for f in range(4):  # a frame's rows at a time: the GEMM's operands stay under 4 GiB
        cols = kernels.im2col_causal(x[2:].contiguous(), (h, w), c, kt=3, ks=3, kpad=2624,
                                     cache=x[:2].contiguous(), row0=f * po, rows=po)
        kernels.gemm_grouped([kernels.Problem(cols, wt, ref[f * po:(f + 1) * po], bias)],
                             kind="bf16")
        del cols
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_conv_causal_refuses_what_it_cannot_run(gpu):
    x = torch.zeros(2, 12, 16, dtype=torch.bfloat16, device=gpu)
    wt = torch.zeros(16, 448, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="overrun"):
        kernels.conv_causal(x, (3, 4), 16, 3, wt, kt=3, ks=3)
    with pytest.raises(ValueError, match="bf16 or fp32"):
        kernels.conv_causal(x.half(), (3, 4), 16, 2, wt.half(), kt=3, ks=3)
    with pytest.raises(ValueError, match="dtype"):
        kernels.conv_causal(x.float(), (3, 4), 16, 2, wt, kt=3, ks=3)
    with pytest.raises(ValueError, match="multiple of 64"):
        kernels.conv_causal(x, (3, 4), 16, 2, wt[:, :440].contiguous(), kt=3, ks=3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("c", [16, 96, 192, 384, 1024])
def test_rms_norm_channels(gpu, dtype, c):
    g = torch.Generator().manual_seed(c)
    x = (torch.randn(777, c + 8, generator=g) * 3).to(dtype)[:, :c]  # strided rows
    x[5] = 0
    gamma = 1 + 0.1 * torch.randn(c, generator=g)
    for silu in (False, True):
        ref = x.float() * c ** 0.5 / x.float().norm(dim=1, keepdim=True).clamp_min(1e-12) * gamma
        ref = F.silu(ref) if silu else ref
        out = kernels.rms_norm_channels(x.to(gpu), gamma.to(gpu), silu=silu)
        assert out.dtype == dtype and torch.equal(out[5].cpu(), torch.zeros(c, dtype=dtype))
        assert rel_l2(out, ref) < (2e-6 if dtype == torch.float32 else 4e-3)


def test_rows_to_planes_clamps_and_keeps_nan(gpu):
    x = torch.randn(100, 4) * 3
    x[7, 1] = float("nan")
    out = kernels.rows_to_planes(x.to(gpu), 3, lo=-1.0, hi=1.0).cpu()
    ref = x[:, :3].t().clamp(-1.0, 1.0)
    assert torch.equal(torch.nan_to_num(out, 9.0), torch.nan_to_num(ref, 9.0))
    assert torch.isnan(out[1, 7])


SMALL = ow.WanVaeShape(base_dim=8, z_dim=16, dim_mult=(1, 2, 4, 4), num_res_blocks=1,
                       temperal_downsample=(False, True, True))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("t,hw", [(3, (4, 6)), (2, (3, 5))])
def test_small_decoder_matches_oracle(gpu, dtype, t, hw, parity):
    """Two temporal upsamplings and one spatial, a resnet with a 1x1 shortcut (16 -> 32
    channels), the mid-block attention over 24 or 15 pixels (15: the scores' key count padded)."""
    print(f"wan vae small {dtype} t={t} {hw}", flush=True)
    store = None if dtype == torch.float32 else dtype
    w = ow.weights(SMALL, 8, store)
    dec = dwan.WanVaeDecoder(_cfg(SMALL), lambda n: w[n], dtype=dtype, device=gpu)
    z = torch.randn(1, 16, t, *hw, generator=torch.Generator().manual_seed(9))
    ref = ow.decode(w, SMALL, z, store=store)
    out = dec.decode(z.to(gpu))
    torch.cuda.synchronize()
    assert out.dtype == dtype and tuple(out.shape) == tuple(ref.shape)
    e = rel_l2(out, ref)
    print(f"  rel L2 {e:.3e}", flush=True)
    bound = 1e-4 if dtype == torch.float32 else 2e-2
    parity(f"small Wan VAE decode {str(dtype)[6:]}, rel L2 vs oracle at the device's rounding "
           "points", e, bound)
    assert e < bound


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_wan_widths_on_a_small_latent_match_oracle(gpu, dtype, parity):
    """Wan 2.2's decoder (384 / 192 / 96 channels) on two 6 x 10 latent frames (5 frames of
    48 x 80); and its mid-block attention alone on a full 60 x 104 latent frame (6240
    pixels, one head of 384 channels)."""
    print(f"wan vae widths {dtype}", flush=True)
    store = None if dtype == torch.float32 else dtype
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    w = ow.weights(ow.WAN_VAE, 10, store)
    dec = dwan.WanVaeDecoder(dwan.WAN_VAE, lambda n: w[n], dtype=dtype, device=gpu)
    z = torch.randn(1, 16, 2, 6, 10, generator=torch.Generator().manual_seed(11))
    ref = ow.decode(w, ow.WAN_VAE, z, store=store)
    out = dec.decode(z.to(gpu))
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, 3, 5, 48, 80)
    e = rel_l2(out, ref)
    print(f"  decode rel L2 {e:.3e}", flush=True)
    parity(f"Wan VAE widths decode {str(dtype)[6:]}, rel L2 vs oracle", e, tol)
    assert e < tol
    r = (lambda x: x) if store is None else (lambda x: x.to(store).float())
    x = r(torch.randn(1, 384, 1, 60, 104, generator=torch.Generator().manual_seed(12)))
    pre = "decoder.mid_block.attentions.0"
    ref = ow.attention(w, pre, x, ow.WAN_VAE, r)
    xd = x[0, :, 0].permute(1, 2, 0).reshape(1, 6240, 384).to(gpu, dtype).contiguous()
    got = dec._attention(pre, dwan._Chunk(xd, 1, (60, 104), 384))
    e = rel_l2(got.data[0].reshape(60, 104, 384).permute(2, 0, 1), ref[0, :, 0])
    print(f"  attention rel L2 {e:.3e}", flush=True)
    assert e < tol


def test_wan_vae_full_decode_480p_81_frames(gpu):
    """Wan 2.2's VAE decoder on a 21 x 60 x 104 latent (81 frames of 480 x 832), random
    weights: bf16 and fp32 finite, in [-1, 1] and bit-identical on a rerun; bf16 within 5e-2 of
    fp32; causal (a change to the last latent frame leaves frames 0..76 bit-identical); the
    first latent frame decoded alone equals frame 0 (Qwen-Image's one-frame decode)."""
    z = torch.randn(1, 16, 21, 60, 104, generator=torch.Generator().manual_seed(13)).to(gpu)
    outs = {}
    for dt in (torch.float32, torch.bfloat16):
        print(f"wan vae full decode {dt}", flush=True)
        dec = dwan.WanVaeDecoder(dwan.WAN_VAE, dwan.random_param_source(dwan.WAN_VAE, 3, gpu),
                                 dtype=dt, device=gpu)
        a = dec.decode(z)
        b = dec.decode(z)
        torch.cuda.synchronize()
        assert tuple(a.shape) == (1, 3, 81, 480, 832)
        assert torch.isfinite(a.float()).all() and a.abs().max() <= 1.0
        assert torch.equal(a, b)
        if dt == torch.bfloat16:
            z2 = z.clone()
            z2[:, :, 20] += 0.5
            c = dec.decode(z2)
            assert torch.equal(c[:, :, :77], a[:, :, :77]) and not torch.equal(c[:, :, 77:], a[:, :, 77:])
            one = dec.decode(z[:, :, :1])
            assert tuple(one.shape) == (1, 3, 1, 480, 832) and torch.equal(one[:, :, 0], a[:, :, 0])
        outs[dt] = a.float()
        del dec
        torch.cuda.empty_cache()
    e = rel_l2(outs[torch.bfloat16], outs[torch.float32])
    print(f"  bf16 vs fp32 rel L2 {e:.3e}", flush=True)
    assert e < 5e-2
