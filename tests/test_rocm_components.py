"""The rocm DiT components and the FLUX pipeline adapter, host side: the safetensors reader,
config mapping, RoPE from the caller's ids and its cache, the prompt-padding trim, and the
life-cycle refusals. The device runs are in test_gpu_components.py."""

import types

import pytest
import torch

from difflet_amd.backends.rocm.component import SafetensorsDir, model_output
from difflet_amd.backends.rocm.flux.transformer import (FluxDiTAdapter,
                                                        RocmFluxTransformerApplication,
                                                        flux_config, flux_pos_embed)
from difflet_amd.backends.rocm.qwen_image.transformer import (
    RocmQwenImageTransformerApplication, qwen_config, trim_text_padding)
from difflet_amd.backends.rocm.wan.transformer import RocmWanTransformerApplication, wan_config
from oracle import ops


def flux_dit_config(**kw):
    """A FluxDiTConfig's fields (difflet/models/flux/dit_config.py:22-49) as a namespace."""
    base = dict(patch_size=1, in_channels=64, out_channels=None, num_layers=19,
                num_single_layers=38, attention_head_dim=128, num_attention_heads=24,
                joint_attention_dim=4096, pooled_projection_dim=768, guidance_embeds=True,
                axes_dims_rope=(16, 56, 56), torch_dtype=torch.bfloat16, image_seq_len=4096)
    base.update(kw)
    return types.SimpleNamespace(**base)


def test_safetensors_dir_reads_single_files_and_indexed_shards(tmp_path):
    import json

    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(0)
    t = {f"blocks.{i}.w": torch.randn(3, 4, generator=g) for i in range(4)}
    one = tmp_path / "one"
    one.mkdir()
    save_file(t, str(one / "diffusion_pytorch_model.safetensors"))
    src = SafetensorsDir(one)
    assert src.keys() == sorted(t) and "blocks.2.w" in src
    assert all(torch.equal(src.get(k), v) for k, v in t.items())
    sharded = tmp_path / "sharded"
    sharded.mkdir()
    names = sorted(t)
    save_file({k: t[k] for k in names[:2]}, str(sharded / "m-00001-of-00002.safetensors"))
    save_file({k: t[k] for k in names[2:]}, str(sharded / "m-00002-of-00002.safetensors"))
    wm = {k: ("m-00001-of-00002.safetensors" if k in names[:2] else "m-00002-of-00002.safetensors")
          for k in names}
    (sharded / "diffusion_pytorch_model.safetensors.index.json").write_text(
        json.dumps({"metadata": {}, "weight_map": wm}))
    src = SafetensorsDir(sharded)
    assert all(torch.equal(src[k], v) for k, v in t.items())
    with pytest.raises(KeyError):
        src.get("blocks.9.w")
    pre = SafetensorsDir(one, prefix="blocks.")
    assert torch.equal(pre.get("1.w"), t["blocks.1.w"])
    with pytest.raises(FileNotFoundError):
        SafetensorsDir(tmp_path / "one" / "..", prefix="")  # a directory with no files of its own


def test_configs_map_the_reference_field_names():
    c = flux_config(flux_dit_config())
    assert (c.hidden, c.heads, c.head_dim, c.n_double, c.n_single, c.in_channels,
            c.out_channels, c.txt_dim, c.pooled_dim, c.guidance) == \
        (3072, 24, 128, 19, 38, 64, 64, 4096, 768, True)
    q = qwen_config(types.SimpleNamespace(
        patch_size=2, in_channels=64, out_channels=16, num_layers=60, attention_head_dim=128,
        num_attention_heads=24, joint_attention_dim=3584, guidance_embeds=False,
        axes_dims_rope=(16, 56, 56)))
    assert (q.hidden, q.mlp, q.n_blocks, q.txt_dim, q.out_channels) == (3072, 12288, 60, 3584, 16)
    wan = types.SimpleNamespace(patch_size=(1, 2, 2), num_attention_heads=40,
                                attention_head_dim=128, in_channels=16, out_channels=16,
                                text_dim=4096, freq_dim=256, ffn_dim=13824, num_layers=40,
                                rope_max_seq_len=1024, cfg_parallel_enabled=False)
    w = wan_config(wan)
    assert (w.hidden, w.ffn, w.n_blocks, w.patch) == (5120, 13824, 40, (1, 2, 2))
    wan.cfg_parallel_enabled = True
    with pytest.raises(NotImplementedError):
        wan_config(wan)


def test_flux_pos_embed_is_the_reference_table():
    """The adapter's table from ids equals the oracle's FluxPosEmbed restatement (pinned by
    its closed form in test_oracle_ops.py) for arbitrary ids, and the fused step's grid table
    for the pipeline's (0, i, j) ids."""
    from difflet_amd.dit.rope import flux_rope_tables

    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 90, (50, 3), generator=g).float()
    c0, s0 = flux_pos_embed(ids, (16, 56, 56))
    c1, s1 = ops.flux_pos_embed(ids, (16, 56, 56))
    assert torch.equal(c0, c1) and torch.equal(s0, s1)
    ids = ops.flux_ids(7, 5, 9)
    c0, s0 = flux_pos_embed(ids, (16, 56, 56))
    c2, s2 = flux_rope_tables(7, (5, 9), device="cpu")
    assert torch.equal(c0, c2) and torch.equal(s0, s2)


def _pipeline_ids(txt_len, h, w):
    """FluxPipeline's ids: text zeros [txt_len, 3]; latent image ids (0, row, column) over the
    packed h x w grid, row-major."""
    img = torch.zeros(h, w, 3)
    img[..., 1] += torch.arange(h)[:, None]
    img[..., 2] += torch.arange(w)[None, :]
    return torch.zeros(txt_len, 3), img.reshape(h * w, 3)


def test_adapter_builds_the_table_from_ids_in_the_model_dtype_and_caches_it():
    app = RocmFluxTransformerApplication(config=flux_dit_config(), device="cpu",
                                         get=lambda n: None)
    ad = FluxDiTAdapter(app)
    txt, img = _pipeline_ids(4, 2, 8)
    cos, sin = ad.rotary_embedding(txt, img)
    ref_c, ref_s = flux_pos_embed(torch.cat([txt, img]), (16, 56, 56))
    assert cos.dtype == torch.float32 and cos.shape == (20, 128)
    assert torch.equal(cos, ref_c.bfloat16().float()) and torch.equal(sin, ref_s.bfloat16().float())
    again = ad.rotary_embedding(txt[None], img[None])  # [1, S, 3] ids as older pipelines pass
    assert again[0] is cos
    txt2, img2 = _pipeline_ids(4, 8, 2)  # same shapes, other grid: not the cached table
    other = ad.rotary_embedding(txt2, img2)
    assert other[0] is not cos and not torch.equal(other[0], cos)


def test_trim_text_padding_follows_the_reference_law():
    x = torch.arange(10.0).view(1, 10, 1)
    y, n = trim_text_padding(x, torch.tensor([True] * 6 + [False] * 4))
    assert n == 6 and torch.equal(y, x[:, :6])
    y, n = trim_text_padding(x, None)
    assert n == 10 and y is x
    y, n = trim_text_padding(x, torch.ones(10, dtype=torch.bool))
    assert n == 10
    with pytest.raises(NotImplementedError):
        trim_text_padding(x, torch.tensor([True, False, True] + [False] * 7))
    with pytest.raises(ValueError):
        trim_text_padding(x, torch.zeros(10, dtype=torch.bool))


def test_components_refuse_before_load_and_off_device():
    with pytest.raises(ValueError):
        RocmFluxTransformerApplication(config=flux_dit_config())  # no path, no get
    with pytest.raises(NotImplementedError):
        RocmFluxTransformerApplication(config=flux_dit_config(torch_dtype=torch.float32),
                                       get=lambda n: None)
    with pytest.raises(ValueError):
        RocmFluxTransformerApplication(config=flux_dit_config(), get=lambda n: None, kind="int4")
    app = RocmFluxTransformerApplication(config=flux_dit_config(), device="cpu",
                                         get=lambda n: None)
    assert not app.is_loaded and app.repeated_blocks() == []
    with pytest.raises(RuntimeError, match="not loaded"):
        app(torch.zeros(1, 4, 64), torch.zeros(1, 2, 4096), torch.zeros(1, 768), torch.zeros(1),
            torch.tensor([3.5]), torch.zeros(6, 128, 2))
    with pytest.raises(RuntimeError, match="ROCm device"):
        app.load()
    ex = app.get_example_inputs()
    assert [tuple(t.shape) for t in ex] == [(1, 4096, 64), (1, 512, 4096), (1, 768), (1,), (1,),
                                           (4608, 128, 2)]
    for cls in (RocmQwenImageTransformerApplication, RocmWanTransformerApplication):
        with pytest.raises(ValueError):
            cls(config=None, device="cpu", get=lambda n: None, kind="fp4")


def test_model_output_has_sample_and_indexes_like_a_tuple():
    t = torch.ones(2)
    out = model_output(t)
    assert out.sample is t and out[0] is t


def test_attention_head_dim_padding_law():
    """Other head dims run the 64 / 128 kernels on zero-padded q, k, v: the padded dimensions
    add exact zeros to every score and give zero output columns, so padding then cutting the
    output back is the unpadded attention (checked here with the fp32 oracle on the CPU)."""
    from difflet_amd.backends.rocm.ops_impl.attention import kernel_head_dim, pad_head_dim
    from oracle import ops

    assert [kernel_head_dim(d) for d in (8, 40, 63, 64, 65, 96, 127, 128)] == \
        [64, 64, 64, 64, 128, 128, 128, 128]
    for bad in (0, 129, 256):
        with pytest.raises(NotImplementedError):
            kernel_head_dim(bad)
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, 2, 33, 40, generator=g) for _ in range(3))
    sc = 40 ** -0.5
    ref = ops.attention(q, k, v, scale=sc)
    qp, kp, vp = (pad_head_dim(t, 64) for t in (q, k, v))
    assert qp.shape[-1] == 64 and torch.equal(qp[..., 40:], torch.zeros_like(qp[..., 40:]))
    out = ops.attention(qp, kp, vp, scale=sc)
    assert torch.equal(out[..., 40:], torch.zeros_like(out[..., 40:]))
    assert torch.allclose(out[..., :40], ref, atol=1e-6, rtol=1e-6)
