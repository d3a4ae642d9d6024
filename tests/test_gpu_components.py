"""The rocm DiT components on the device: the FLUX adapter driven as FluxPipeline drives it
(packed latents, text and image ids, guidance, return_dict) against the oracle's forward, and
the FLUX, Qwen-Image and Wan components built from diffusers safetensors directories against
the fused steps built from the same tensors."""

import types

import pytest
import torch

from difflet_amd.backends.rocm.flux.transformer import (FluxDiTAdapter,
                                                        RocmFluxTransformerApplication)
from difflet_amd.backends.rocm.qwen_image.transformer import RocmQwenImageTransformerApplication
from difflet_amd.backends.rocm.wan.transformer import RocmWanTransformerApplication
from oracle import flux as oflux

pytestmark = pytest.mark.gpu

SEED = 2024


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def flux_dit_config(**kw):
    base = dict(patch_size=1, in_channels=64, out_channels=None, num_layers=19,
                num_single_layers=38, attention_head_dim=128, num_attention_heads=24,
                joint_attention_dim=4096, pooled_projection_dim=768, guidance_embeds=True,
                axes_dims_rope=(16, 56, 56), torch_dtype=torch.bfloat16, image_seq_len=4096)
    base.update(kw)
    return types.SimpleNamespace(**base)


def pack_latents(latents):
    """FluxPipeline._pack_latents: [B, C, H, W] -> [B, H/2 * W/2, 4C], 2 x 2 patches row-major,
    features in (c, dy, dx) order."""
    b, c, h, w = latents.shape
    x = latents.view(b, c, h // 2, 2, w // 2, 2).permute(0, 2, 4, 1, 3, 5)
    return x.reshape(b, (h // 2) * (w // 2), c * 4)


def pipeline_ids(txt_len, h, w):
    img = torch.zeros(h, w, 3)
    img[..., 1] += torch.arange(h)[:, None]
    img[..., 2] += torch.arange(w)[None, :]
    return torch.zeros(txt_len, 3), img.reshape(h * w, 3)


def test_flux_adapter_as_the_pipeline_calls_it_matches_the_oracle(gpu, parity):
    """2 double + 2 single blocks at FLUX width. Latents [1, 16, 24, 40] packed to a 12 x 20
    grid (a non-square one, so rows and columns of the ids must not be swapped) with 64 text
    tokens; timestep t / 1000, guidance 3.5. The oracle takes the same ids and the table
    rounded to bf16, as the reference adapter stacks it (bf16: rel L2 <= 1e-2)."""
    print("flux adapter 2 + 2 blocks, 12 x 20 grid + 64 text", flush=True)
    shape = oflux.FluxShape(n_double=2, n_single=2)
    ew = oflux.embed_weights(shape, SEED)
    dws = [oflux.double_block_weights(shape, SEED, i) for i in range(2)]
    sws = [oflux.single_block_weights(shape, SEED, i) for i in range(2)]
    w = dict(ew)
    for i in range(2):
        w.update({f"transformer_blocks.{i}.{k}": v for k, v in dws[i].items()})
        w.update({f"single_transformer_blocks.{i}.{k}": v for k, v in sws[i].items()})
    cfg = flux_dit_config(num_layers=2, num_single_layers=2, image_seq_len=240)
    app = RocmFluxTransformerApplication(config=cfg, device=gpu, get=lambda n: w[n])
    app.load()
    adapter = FluxDiTAdapter(app)
    g = torch.Generator().manual_seed(SEED)
    latents = pack_latents(torch.randn(1, 16, 24, 40, generator=g)).bfloat16()
    text = torch.randn(1, 64, 4096, generator=g).bfloat16()
    pooled = torch.randn(1, 768, generator=g).bfloat16()
    t = torch.tensor([0.6180])
    txt_ids, img_ids = pipeline_ids(64, 12, 20)
    out = adapter(hidden_states=latents.to(gpu), encoder_hidden_states=text.to(gpu),
                  pooled_projections=pooled.to(gpu), timestep=t.to(gpu),
                  img_ids=img_ids.to(gpu), txt_ids=txt_ids.to(gpu), guidance=torch.tensor([3.5],
                  device=gpu), joint_attention_kwargs=None, return_dict=False)[0]
    torch.cuda.synchronize()
    ref = oflux.forward(shape, SEED, latents.float(), text.float(), pooled.float(), t,
                        torch.tensor([3.5]), (12, 20), weights=(ew, dws, sws),
                        model_dtype=torch.bfloat16, rope_dtype=torch.bfloat16)
    e = rel_l2(out, ref)
    print(f"adapter step rel L2 vs fp32 oracle {e:.3e}", flush=True)
    parity("FluxDiTAdapter 2 + 2 block step from pipeline ids, rel L2 vs fp32 oracle", e, 1e-2)
    assert out.shape == (1, 240, 64) and out.dtype == torch.bfloat16
    assert e < 1e-2
    # the second step reuses the cached table and gives the same output; a batch of two
    # requests equals the two requests run alone
    again = adapter(latents.to(gpu), text.to(gpu), pooled.to(gpu), t.to(gpu), img_ids.to(gpu),
                    txt_ids.to(gpu), 3.5).sample
    both = adapter(torch.cat([latents, latents.flip(1)]).to(gpu), text.repeat(2, 1, 1).to(gpu),
                   pooled.repeat(2, 1).to(gpu), torch.tensor([0.618, 0.25], device=gpu),
                   img_ids.to(gpu), txt_ids.to(gpu), 3.5).sample
    second = adapter(latents.flip(1).to(gpu), text.to(gpu), pooled.to(gpu),
                     torch.tensor([0.25], device=gpu), img_ids.to(gpu), txt_ids.to(gpu),
                     3.5).sample
    torch.cuda.synchronize()
    assert torch.equal(again, out)
    assert torch.equal(both[0], out[0]) and torch.equal(both[1], second[0])


def _save(tmp_path, name, tensors):
    from safetensors.torch import save_file

    d = tmp_path / name / "transformer"
    d.mkdir(parents=True)
    save_file({k: v.contiguous() for k, v in tensors.items()},
              str(d / "diffusion_pytorch_model.safetensors"))
    return d


def _toy(shapes, seed):
    g = torch.Generator().manual_seed(seed)
    return {n: (torch.ones(s) if n.endswith("norm.weight") or ".norm_" in n
                else torch.randn(s, generator=g) * 0.02).to(torch.bfloat16)
            for n, s in sorted(shapes.items())}


def test_flux_component_from_a_diffusers_directory(gpu, tmp_path):
    """A toy FLUX (hidden 512) saved under diffusers' names: the component reading the
    directory equals the fused step built from the same tensors, bit for bit."""
    from difflet_amd.dit.flux import FluxConfig, FluxDiT, flux_param_shapes

    print("flux component from a safetensors directory", flush=True)
    fc = FluxConfig(hidden=512, heads=4, n_double=1, n_single=1, txt_dim=256, pooled_dim=128)
    src = _toy(flux_param_shapes(fc), 3)
    d = _save(tmp_path, "flux", src)
    cfg = flux_dit_config(num_layers=1, num_single_layers=1, num_attention_heads=4,
                          joint_attention_dim=256, pooled_projection_dim=128, image_seq_len=64)
    app = RocmFluxTransformerApplication(model_path=str(d), config=cfg, device=gpu)
    app.load()
    ref_dit = FluxDiT(fc, lambda n: src[n], device=gpu)
    g = torch.Generator().manual_seed(4)
    lat = torch.randn(1, 64, 64, generator=g).to(gpu)
    txt = torch.randn(1, 32, 256, generator=g).to(gpu)
    pooled = torch.randn(1, 128, generator=g).to(gpu)
    t, gd = torch.tensor([0.4], device=gpu), torch.tensor([3.5], device=gpu)
    txt_ids, img_ids = pipeline_ids(32, 8, 8)
    out = FluxDiTAdapter(app)(lat, txt, pooled, t, img_ids, txt_ids, gd).sample
    cos, sin = FluxDiTAdapter(app).rotary_embedding(txt_ids, img_ids)
    ref = ref_dit.forward_rope(lat, txt, pooled, t.bfloat16(), gd, cos, sin)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out, ref)


def test_qwen_component_trims_a_right_padded_prompt(gpu, tmp_path):
    """A toy Qwen-Image (hidden 512) from its directory: a prompt right-padded to 48 rows with
    the pipeline's mask gives the output of the 29-row prompt alone, and of the fused step's
    text_valid_len bound."""
    from difflet_amd.dit.qwen import QwenConfig, QwenImageDiT, qwen_param_shapes

    print("qwen component, right-padded prompt", flush=True)
    qc = QwenConfig(hidden=512, heads=4, mlp=2048, n_blocks=2, txt_dim=256)
    src = _toy(qwen_param_shapes(qc), 5)
    d = _save(tmp_path, "qwen", src)
    cfg = types.SimpleNamespace(patch_size=2, in_channels=64, out_channels=64, num_layers=2,
                                attention_head_dim=128, num_attention_heads=4,
                                joint_attention_dim=256, guidance_embeds=False,
                                axes_dims_rope=(16, 56, 56), torch_dtype=torch.bfloat16,
                                packed_height=6, packed_width=10, image_seq_len=60,
                                text_seq_len=48, batch_size=1)
    app = RocmQwenImageTransformerApplication(model_path=str(d), config=cfg, device=gpu,
                                              kind="bf16")
    app.load()
    g = torch.Generator().manual_seed(6)
    lat = torch.randn(1, 60, 64, generator=g).to(gpu)
    txt = torch.randn(1, 48, 256, generator=g).to(gpu)
    mask = torch.zeros(1, 48, dtype=torch.bool)
    mask[:, :29] = True
    t = torch.tensor([0.3], device=gpu)
    out = app(lat, t, txt, mask.to(gpu))
    dit = QwenImageDiT(qc, lambda n: src[n], kind="bf16", device=gpu)
    alone = dit.forward(lat, txt[:, :29], t, (6, 10))
    bounded = dit.forward(lat, txt, t, (6, 10), text_valid_len=29)
    torch.cuda.synchronize()
    assert out.shape == (1, 60, 64) and torch.isfinite(out.float()).all()
    assert torch.equal(out, alone) and torch.equal(out, bounded)


def test_wan_component_from_a_diffusers_directory(gpu, tmp_path):
    """A toy Wan expert (hidden 512) under diffusers' FFN names (ffn.net.0.proj / ffn.net.2):
    the component equals the fused step on the module's names, and a CFG pair [uncond, cond]
    equals its two requests run alone."""
    from difflet_amd.dit.wan import WanConfig, WanDiT, checkpoint_key, wan_param_shapes

    print("wan component from a safetensors directory", flush=True)
    wc = WanConfig(hidden=512, heads=4, ffn=1536, n_blocks=2, text_dim=256)
    src = _toy(wan_param_shapes(wc), 7)
    d = _save(tmp_path, "wan", {checkpoint_key(n): t for n, t in src.items()})
    cfg = types.SimpleNamespace(patch_size=(1, 2, 2), num_attention_heads=4, attention_head_dim=128,
                                in_channels=16, out_channels=16, text_dim=256, freq_dim=256,
                                ffn_dim=1536, num_layers=2, rope_max_seq_len=1024,
                                torch_dtype=torch.bfloat16)
    app = RocmWanTransformerApplication(model_path=str(d), config=cfg, device=gpu)
    app.load()
    dit = WanDiT(wc, lambda n: src[n], device=gpu)
    g = torch.Generator().manual_seed(8)
    lat = torch.randn(2, 16, 2, 8, 8, generator=g).to(gpu)
    txt = torch.randn(2, 24, 256, generator=g).to(gpu)
    t = torch.tensor([700.0], device=gpu)
    out = app(lat, t, txt)
    ref0 = dit.forward(lat[:1], t, txt[:1])
    ref1 = dit.forward(lat[1:], t, txt[1:])
    torch.cuda.synchronize()
    assert out.shape == (2, 16, 2, 8, 8) and torch.isfinite(out.float()).all()
    assert torch.equal(out[:1], ref0) and torch.equal(out[1:], ref1)
