"""Pins of the Wan VAE decoder oracle (oracle/wan_vae.py) and the host side of the device
decoder (difflet_amd/vae/wan.py), on the CPU.

The reference decoder cannot be imported here (it imports diffusers, absent), so the oracle is
pinned by: the reference's own tests of the decoder config, key layout and tiny forward
(tests/unit/models/wan/test_modeling_wan_vae.py:37-143); the chunked decode against an
independent whole-sequence statement of the same decoder; the "Rep" rule of the first time
convolution and the interleave order, by hand-made weights with a closed-form output; causality
(later latent frames never change earlier output frames); the first frame alone equals the first
frame of a longer decode (Qwen-Image's one-frame decode); WanRMSNorm against its closed form;
the attention block against torch's SDPA. Planted mistakes (symmetric temporal padding, the
time convolution reading the first frame, swapped interleave halves) fail these checks."""

import math

import pytest
import torch
import torch.nn.functional as F

from difflet_amd.vae import wan as dwan
from oracle import wan_vae as ow


def rel_l2(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


TINY = ow.WanVaeShape(base_dim=8, z_dim=4, dim_mult=(1, 2), num_res_blocks=1,
                      temperal_downsample=(True,))
# two temporal upsamplings and one spatial-only, as Wan's (1, 2, 4, 4) has, at small widths
SMALL = ow.WanVaeShape(base_dim=4, z_dim=8, dim_mult=(1, 2, 4, 4), num_res_blocks=1,
                       temperal_downsample=(False, True, True))


def _z(shape, t, h, w, seed=1):
    return torch.randn(1, shape.z_dim, t, h, w, generator=torch.Generator().manual_seed(seed))


def test_wan22_defaults_and_plan():
    """test_wan_vae_decoder_config_defaults_match_wan22 (reference test :37-50) and the up-block
    plan of modeling_vae.py:436-456 at Wan's widths."""
    cfg = dwan.WanVaeConfig()
    assert (cfg.base_dim, cfg.decoder_base_dim, cfg.z_dim) == (96, 96, 16)
    assert cfg.dim_mult == (1, 2, 4, 4) and cfg.num_res_blocks == 2 and cfg.attn_scales == ()
    assert cfg.temperal_downsample == (False, True, True)
    assert cfg.temperal_upsample == (True, True, False)
    assert (cfg.scale_factor_temporal, cfg.scale_factor_spatial) == (4, 8)
    assert ow.WAN_VAE.dims == cfg.dims == [384, 384, 384, 192, 96]
    assert ow.plan(ow.WAN_VAE) == dwan.plan(cfg) == [
        (0, 384, 384, "upsample3d"), (1, 192, 384, "upsample3d"), (2, 192, 192, "upsample2d"),
        (3, 96, 96, None)]


def test_config_from_diffusers_dict_and_refusals():
    """Reference tests :53-79: unknown keys dropped; is_residual, a patch size and a mismatched
    temporal list refused with the reference's error types."""
    cfg = dwan.WanVaeConfig.from_diffusers_dict(
        {"base_dim": 96, "z_dim": 16, "dim_mult": [1, 2, 4, 4], "num_res_blocks": 2,
         "_class_name": "AutoencoderKLWan", "_diffusers_version": "0.38.0"})
    assert cfg.base_dim == 96 and cfg.z_dim == 16 and cfg.dim_mult == (1, 2, 4, 4)
    with pytest.raises(NotImplementedError, match="is_residual"):
        dwan.WanVaeConfig(is_residual=True)
    with pytest.raises(NotImplementedError, match="patchified"):
        dwan.WanVaeConfig(patch_size=2)
    with pytest.raises(ValueError, match="temperal_downsample"):
        dwan.WanVaeConfig(dim_mult=(1, 2, 4), temperal_downsample=(True,))


def test_key_layout_matches_the_reference_decoder():
    """Reference test :97-121 on its tiny config; the device decoder and the oracle name and
    shape every parameter alike, at the tiny config and at Wan's."""
    keys = dict(ow.param_shapes(TINY))
    for k in ("post_quant_conv.weight", "decoder.conv_in.weight",
              "decoder.mid_block.resnets.0.conv1.weight", "decoder.up_blocks.0.resnets.0.conv1.weight",
              "decoder.norm_out.gamma", "decoder.conv_out.weight"):
        assert k in keys
    assert not any(k.startswith(("encoder.", "quant_conv.")) for k in keys)
    for shape in (TINY, ow.WAN_VAE):
        cfg = dwan.WanVaeConfig(base_dim=shape.base_dim, z_dim=shape.z_dim,
                                dim_mult=shape.dim_mult, num_res_blocks=shape.num_res_blocks,
                                temperal_downsample=shape.temperal_downsample)
        assert dwan.param_shapes(cfg) == dict(ow.param_shapes(shape))


def test_tiny_forward_shape_and_clamp():
    """Reference test :124-143: two latent frames, one temporal upsampling -> 1 + 2 frames at
    2x, inside [-1, 1]."""
    w = ow.weights(TINY, 0)
    out = ow.decode(w, TINY, torch.randn(1, 4, 2, 4, 4, generator=torch.Generator().manual_seed(0)))
    assert out.shape == (1, 3, 3, 8, 8)
    assert out.min() >= -1.0 and out.max() <= 1.0


@pytest.mark.parametrize("store", [None, torch.bfloat16])
def test_chunked_decode_equals_the_whole_sequence_statement(store):
    """Two temporal upsamplings: 3 latent frames -> 9 frames at 8x."""
    w = ow.weights(SMALL, 2, store)
    z = _z(SMALL, 3, 3, 4)
    a = ow.decode(w, SMALL, z, store=store)
    b = ow.decode_sequence(w, SMALL, z, store=store)
    assert a.shape == (1, 3, 9, 24, 32)
    # fp32: summation order only; bf16: roundings flipped by that order, carried through 30 layers
    assert rel_l2(a, b) < (1e-5 if store is None else 1e-2)


def test_causality_and_the_first_frame_alone():
    w = ow.weights(SMALL, 3)
    z = _z(SMALL, 3, 3, 4, seed=4)
    base = ow.decode(w, SMALL, z)
    z2 = z.clone()
    z2[:, :, 2] += 1.0
    moved = ow.decode(w, SMALL, z2)
    # chunks 0 and 1 give frames 0..4; chunk 2 frames 5..8
    assert torch.equal(moved[:, :, :5], base[:, :, :5])
    assert not torch.allclose(moved[:, :, 5:], base[:, :, 5:])
    one = ow.decode(w, SMALL, z[:, :, :1])
    assert one.shape[2] == 1 and torch.equal(one[:, :, 0], base[:, :, 0])


def test_planted_symmetric_time_padding_breaks_causality(monkeypatch):
    w = ow.weights(SMALL, 3)
    z = _z(SMALL, 3, 3, 4, seed=4)
    real = ow.causal_conv

    def symmetric(x, wt, b, cache=None):
        if wt.shape[2] == 1 or cache is not None:
            return real(x, wt, b, cache)
        return F.conv3d(F.pad(x, (wt.shape[3] // 2,) * 4 + (1, 1)), wt, b)

    monkeypatch.setattr(ow, "causal_conv", symmetric)
    a = ow.decode_sequence(w, SMALL, z)
    z2 = z.clone()
    z2[:, :, 2] += 1.0
    b = ow.decode_sequence(w, SMALL, z2)
    assert not torch.allclose(a[:, :, :5], b[:, :, :5])


def _time_walk(x_frames, c, swap=False, first_reads_x0=False, monkeypatch=None):
    """The first upsample3d resampler of a walk over single-frame chunks, its spatial
    convolution replaced by the identity: time-conv output channels [0, C) take the previous
    frame (tap dt = 1), [C, 2C) the current one (dt = 2)."""
    wt = torch.zeros(2 * c, c, 3, 1, 1)
    for o in range(c):
        wt[o, o, 1] = 1.0
        wt[c + o, o, 2] = 1.0
    if swap:
        wt = torch.cat([wt[c:], wt[:c]])
    w = {"u.time_conv.weight": wt, "u.time_conv.bias": torch.zeros(2 * c)}
    monkeypatch.setattr(ow, "spatial_upsample", lambda w_, pre, x, r: x)
    cache: dict = {}
    if first_reads_x0:  # the mistake: chunk 0 feeds the time cache as a regular convolution
        cache["u.time_conv"] = x_frames[:, :, :1]
    walk = ow._Walk(w, SMALL, cache, lambda t: t)
    outs = [walk.resample("u", "upsample3d", x_frames[:, :, i:i + 1]) for i in range(x_frames.shape[2])]
    return torch.cat(outs, dim=2)


def test_first_time_convolution_reads_zeros_and_interleaves_in_order(monkeypatch):
    """Chunk 0 passes through; chunk 1's time convolution sees zeros before it (the reference's
    "Rep" cache), so with the taps above the frames are x0, 0, x1, x1, x2, x2, x3."""
    c = 2
    x = torch.randn(1, c, 4, 2, 2, generator=torch.Generator().manual_seed(6))
    out = _time_walk(x, c, monkeypatch=monkeypatch)
    want = torch.stack([x[:, :, 0], torch.zeros_like(x[:, :, 0]), x[:, :, 1], x[:, :, 1],
                        x[:, :, 2], x[:, :, 2], x[:, :, 3]], dim=2)
    assert torch.equal(out, want)
    # the whole-sequence statement agrees (frames 1.. with two zero frames before frame 1)
    wt = torch.zeros(2 * c, c, 3, 1, 1)
    for o in range(c):
        wt[o, o, 1] = 1.0
        wt[c + o, o, 2] = 1.0
    seq = ow.interleave_time(ow.causal_conv(x[:, :, 1:], wt, torch.zeros(2 * c)))
    assert torch.equal(torch.cat([x[:, :, :1], seq], dim=2), want)
    # planted: swapped interleave halves, or chunk 1 reading x0 before it
    assert not torch.equal(_time_walk(x, c, swap=True, monkeypatch=monkeypatch), want)
    assert not torch.equal(_time_walk(x, c, first_reads_x0=True, monkeypatch=monkeypatch), want)


def test_rms_norm_closed_form():
    """F.normalize(x) sqrt(C) gamma = x rsqrt(mean(x^2)) gamma, and a zero pixel stays zero."""
    x = torch.randn(2, 24, 3, 5, 5, generator=torch.Generator().manual_seed(7))
    x[0, :, 1, 2, 2] = 0.0
    g = 1 + 0.1 * torch.randn(24, 1, 1, 1, generator=torch.Generator().manual_seed(8))
    got = ow.rms_norm(x, g, ow.WAN_VAE)
    want = x * torch.rsqrt((x * x).mean(dim=1, keepdim=True)) * g
    want[0, :, 1, 2, 2] = 0.0
    assert rel_l2(got, want) < 1e-6 and torch.equal(got[0, :, 1, 2, 2], torch.zeros(24))


def test_attention_block_is_sdpa_with_residual():
    shape = ow.WanVaeShape(base_dim=4)
    w = ow.weights(ow.WanVaeShape(base_dim=4), 9)
    pre = "decoder.mid_block.attentions.0"
    c = shape.dims[0]
    x = torch.randn(1, c, 2, 3, 5, generator=torch.Generator().manual_seed(10))
    got = ow.attention(w, pre, x, shape, lambda t: t)
    for f in range(2):
        fr = x[:, :, f]
        n = ow.rms_norm(fr, w[f"{pre}.norm.gamma"], shape)
        qkv = F.conv2d(n, w[f"{pre}.to_qkv.weight"], w[f"{pre}.to_qkv.bias"])
        qkv = qkv.reshape(1, 3 * c, 15).transpose(1, 2)
        q, k, v = qkv.chunk(3, dim=-1)
        o = F.scaled_dot_product_attention(q[:, None], k[:, None], v[:, None])[:, 0]
        o = F.conv2d(o.transpose(1, 2).reshape(1, c, 3, 5), w[f"{pre}.proj.weight"],
                     w[f"{pre}.proj.bias"])
        assert rel_l2(got[:, :, f], o + fr) < 1e-6


def test_packed_weights_times_causal_im2col_rows_are_the_convolution():
    """The device decoder's weight packing and its im2col column order ((dt, ky, kx, c)),
    restated on the CPU, give the causal convolution with a cache."""
    g = torch.Generator().manual_seed(11)
    cin, cout, t, h, w_ = 8, 12, 2, 4, 5
    wt, b = torch.randn(cout, cin, 3, 3, 3, generator=g), torch.randn(cout, generator=g)
    x, cache = torch.randn(1, cin, t, h, w_, generator=g), torch.randn(1, cin, 2, h, w_, generator=g)
    want = ow.causal_conv(x, wt, b, cache)
    cv = dwan.pack_conv(wt, b, 64, torch.float32)
    seq = torch.cat([cache, x], dim=2)[0]  # [C, 2 + t, h, w]
    pad = F.pad(seq, (1, 1, 1, 1))
    rows = []
    for f in range(t):
        taps = [pad[:, f + dt, ky:ky + h, kx:kx + w_] for dt in range(3) for ky in range(3)
                for kx in range(3)]
        rows.append(torch.stack(taps, 0).permute(2, 3, 0, 1).reshape(h * w_, 27 * cin))
    a = F.pad(torch.cat(rows), (0, cv.kpad - 27 * cin))
    got = (a @ cv.w.T + cv.b)[:, :cout]
    assert rel_l2(got, want[0].permute(1, 2, 3, 0).reshape(t * h * w_, cout)) < 1e-6


def test_denormalize():
    z = torch.randn(1, 2, 1, 1, 1, generator=torch.Generator().manual_seed(12))
    out = ow.denormalize(z, [0.5, -1.0], [2.0, 3.0])
    assert torch.allclose(out.flatten(), z.flatten() * torch.tensor([2.0, 3.0]) + torch.tensor([0.5, -1.0]))
    assert torch.equal(ow.denormalize(z, [], []), z)
    assert math.isclose(float(ow.denormalize(z, None, None).sum()), float(z.sum()))
