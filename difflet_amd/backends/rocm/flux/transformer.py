"""The FLUX DiT as a rocm GPU component, and the adapter with the transformer interface
FluxPipeline calls: the load-time module swap of docs/design/gpu_backend.md:36-40 for FLUX,
replacing difflet/backends/cuda/flux/transformer.py:31-221.

`RocmFluxTransformerApplication` builds the fused step (difflet_amd.dit.flux.FluxDiT) from a
diffusers `transformer/` directory, whose parameter names it reads as they are (the fused step
keeps proj_out whole, so the reference's convert_flux_hf_state_dict split is not needed), and
runs it with the CUDA component's forward signature: (hidden_states, encoder_hidden_states,
pooled_projections, timestep, guidance, image_rotary_emb), image_rotary_emb the stacked
[S, head_dim, 2] (cos, sin) table. `FluxDiTAdapter` takes FluxPipeline's call (ids instead of a
table, optional guidance, return_dict), builds the table from the caller's ids with
FluxPosEmbed's law (difflet/layers/embeddings.py:148-244: fp32 positions, float64 frequencies,
repeat-interleaved) cast to the model dtype as the reference adapter does (:168-188), and
caches it per ids.
"""

from __future__ import annotations

from contextlib import contextmanager

import torch

from difflet_amd.backends.rocm.component import RocmComponent, model_output

# FluxPipeline's T5 prompt length (max_sequence_length), the shape of the example inputs
TEXT_SEQ_LEN = 512
ROPE_THETA = 10000


def flux_config(dit_config):
    """difflet_amd.dit.flux.FluxConfig from a FluxDiTConfig (difflet/models/flux/
    dit_config.py:22-49; read by attribute name)."""
    from difflet_amd.dit.flux import FluxConfig

    c = dit_config
    in_ch = int(c.in_channels)
    out_ch = getattr(c, "out_channels", None)
    return FluxConfig(hidden=int(c.num_attention_heads) * int(c.attention_head_dim),
                      heads=int(c.num_attention_heads), head_dim=int(c.attention_head_dim),
                      n_double=int(c.num_layers), n_single=int(c.num_single_layers),
                      in_channels=in_ch, out_channels=int(out_ch) if out_ch else in_ch,
                      txt_dim=int(c.joint_attention_dim),
                      pooled_dim=int(c.pooled_projection_dim),
                      axes=tuple(getattr(c, "axes_dims_rope", (16, 56, 56))),
                      guidance=bool(c.guidance_embeds))


def flux_pos_embed(ids: torch.Tensor, axes_dim, theta: float = ROPE_THETA):
    """FluxPosEmbed.forward (difflet/layers/embeddings.py:148-176): per axis i, angles
    pos_i * theta^(-2j/dim_i) with pos the fp32 ids and float64 frequencies, cos and sin each
    repeated for the interleaved pair, concatenated over the axes; fp32 [S, sum(axes_dim)]."""
    pos = ids.float()
    cos, sin = [], []
    for i, dim in enumerate(axes_dim):
        freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64,
                                              device=ids.device)[: dim // 2] / dim))
        ang = torch.outer(pos[:, i], freqs)
        cos.append(ang.cos().repeat_interleave(2, dim=1).float())
        sin.append(ang.sin().repeat_interleave(2, dim=1).float())
    return torch.cat(cos, dim=-1), torch.cat(sin, dim=-1)


class RocmFluxTransformerApplication(RocmComponent):
    """FLUX's DiT on one MI355X. `kind` picks the block linears' format: "bf16", "fp8"
    (per-channel weights, per-token activations) or "mx" (MXFP8); `quantized_path` loads a
    quantized directory (difflet_amd.quant.checkpoint) instead, its format deciding the kind.
    `fuse_proj_out` is accepted for the reference's signature: the single block's proj_out
    always runs as one GEMM here."""

    def __init__(self, *, model_path=None, config, device=None, torch_compile: bool = False,
                 fuse_proj_out: bool = False, kind: str = "bf16", quantized_path=None,
                 get=None):
        super().__init__(model_path=model_path if quantized_path is None else quantized_path,
                         config=config, device=device, torch_compile=torch_compile, get=get)
        if kind not in ("bf16", "fp8", "mx"):
            raise ValueError(f"kind must be 'bf16', 'fp8' or 'mx', got {kind!r}")
        self.kind = kind
        self.quantized_path = quantized_path
        self.fuse_proj_out = bool(fuse_proj_out)
        self.cfg = flux_config(config)

    def build_module(self):
        from difflet_amd.dit.flux import FluxDiT

        if self.quantized_path is not None:
            return FluxDiT.from_quantized_dir(self.cfg, self.quantized_path, device=self.device)
        return FluxDiT(self.cfg, self.weight_source(), kind=self.kind, device=self.device)

    def get_example_inputs(self) -> tuple:
        c = self.dit_config
        dt = self.dtype
        s_img = int(c.image_seq_len)
        guidance = (torch.tensor([3.5], dtype=dt) if c.guidance_embeds
                    else torch.tensor([], dtype=dt))
        return (torch.zeros(1, s_img, int(c.in_channels), dtype=dt),
                torch.zeros(1, TEXT_SEQ_LEN, int(c.joint_attention_dim), dtype=dt),
                torch.zeros(1, int(c.pooled_projection_dim), dtype=dt),
                torch.zeros(1, dtype=dt), guidance,
                torch.zeros(TEXT_SEQ_LEN + s_img, int(c.attention_head_dim), 2, dtype=dt))

    def forward(self, hidden_states, encoder_hidden_states, pooled_projections, timestep,
                guidance, image_rotary_emb):
        dit = self._require_loaded()
        if image_rotary_emb.dim() != 3 or image_rotary_emb.shape[-1] != 2:
            raise ValueError("image_rotary_emb must be the stacked [S, head_dim, 2] (cos, sin)")
        table = image_rotary_emb.to(self.device)
        cos = table[..., 0].float().contiguous()
        sin = table[..., 1].float().contiguous()
        return self._run(dit, hidden_states, encoder_hidden_states, pooled_projections, timestep,
                         guidance, cos, sin)

    def _run(self, dit, hidden_states, encoder_hidden_states, pooled_projections, timestep,
             guidance, cos, sin):
        """The fused step per request of the batch (it runs one request per launch sequence),
        outputs stacked: [B, S_img, out_ch] in the model dtype."""
        dev = self.device
        b = hidden_states.shape[0]
        per = lambda t: t.reshape(-1).expand(b) if t.numel() == 1 else t.reshape(b)  # noqa: E731
        timestep = per(timestep)
        if self.cfg.guidance:
            if guidance is None or guidance.numel() == 0:
                raise ValueError("this FLUX model embeds guidance: pass a guidance value")
            guidance = per(guidance)
        else:
            guidance = torch.zeros(b)
        outs = [dit.forward_rope(hidden_states[i:i + 1].to(dev),
                                 encoder_hidden_states[i:i + 1].to(dev),
                                 pooled_projections[i:i + 1].to(dev), timestep[i:i + 1].to(dev),
                                 guidance[i:i + 1].to(dev), cos, sin) for i in range(b)]
        return outs[0] if b == 1 else torch.cat(outs, dim=0)


class FluxDiTAdapter(torch.nn.Module):
    """FluxPipeline's transformer interface over a loaded RocmFluxTransformerApplication
    (difflet/backends/cuda/flux/transformer.py:138-221): it reads `config.in_channels`,
    `config.guidance_embeds` and `dtype`, enters `cache_context(name)`, and calls the
    transformer with `txt_ids` / `img_ids`; the table is built here from the ids, cast to the
    model dtype, and cached for the ids of the last call (the denoising loop passes the same
    ids every step)."""

    def __init__(self, app: RocmFluxTransformerApplication):
        super().__init__()
        self.app = app
        self.config = app.dit_config
        self.dtype = app.dtype
        self.axes_dims_rope = tuple(getattr(self.config, "axes_dims_rope", (16, 56, 56)))
        self._rope_cache = None  # (shape key, txt_ids, img_ids, (cos, sin))

    @property
    def device(self) -> torch.device:
        return self.app.device

    @contextmanager
    def cache_context(self, name: str):
        """FluxPipeline enters this around each forward; nothing is cached across it here."""
        del name
        yield

    def rotary_embedding(self, txt_ids: torch.Tensor, img_ids: torch.Tensor):
        """(cos, sin) fp32 [S_txt + S_img, head_dim] on the device, the values of the
        reference's stacked table in the model dtype, for these ids. A cached table is reused
        only for equal ids (equal shapes are not enough: a 2x8 and an 8x2 grid differ)."""
        if txt_ids.ndim == 3:
            txt_ids = txt_ids[0]
        if img_ids.ndim == 3:
            img_ids = img_ids[0]
        key = (tuple(txt_ids.shape), tuple(img_ids.shape))
        c = self._rope_cache
        if c is not None and c[0] == key and torch.equal(c[1], txt_ids.cpu()) \
                and torch.equal(c[2], img_ids.cpu()):
            return c[3]
        ids = torch.cat((txt_ids, img_ids), dim=0).cpu()
        cos, sin = flux_pos_embed(ids, self.axes_dims_rope)
        dev = self.app.device
        table = (cos.to(self.dtype).float().to(dev).contiguous(),
                 sin.to(self.dtype).float().to(dev).contiguous())
        self._rope_cache = (key, txt_ids.cpu().clone(), img_ids.cpu().clone(), table)
        return table

    def forward(self, hidden_states, encoder_hidden_states=None, pooled_projections=None,
                timestep=None, img_ids=None, txt_ids=None, guidance=None,
                joint_attention_kwargs=None, return_dict=True, **ignored):
        del joint_attention_kwargs, ignored
        dit = self.app._require_loaded()
        dev = self.app.device
        if guidance is not None and not isinstance(guidance, torch.Tensor):
            guidance = torch.tensor([guidance], dtype=self.dtype, device=dev)
        elif guidance is not None:
            guidance = guidance.to(self.dtype)
        cos, sin = self.rotary_embedding(txt_ids, img_ids)
        out = self.app._run(dit, hidden_states, encoder_hidden_states, pooled_projections,
                            timestep.to(self.dtype), guidance, cos, sin)
        if not return_dict:
            return (out,)
        return model_output(out)


__all__ = ["FluxDiTAdapter", "RocmFluxTransformerApplication", "TEXT_SEQ_LEN", "flux_config",
           "flux_pos_embed"]
