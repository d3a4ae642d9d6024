"""One Wan DiT expert as a rocm GPU component, replacing difflet/backends/cuda/wan/
transformer.py:24-127 (the load-time module swap of docs/design/gpu_backend.md:36-40 for Wan).

`RocmWanTransformerApplication` builds the fused step (difflet_amd.dit.wan.WanDiT) from one
expert's diffusers directory (`transformer/` or `transformer_2/`), mapping the module's FFN
names to the checkpoint's (net_in / net_out are ffn.net.0.proj / ffn.net.2,
difflet/models/wan/dit_config.py:126-139), and runs it with the CUDA component's forward
signature: (hidden_states [B, C, F, H, W], timestep [B] in 0 .. 1000, encoder_hidden_states
[B, S_txt, text_dim]). A batch (CFG's [uncond, cond] pair) runs one request after the other.
CFG-parallel across two GPUs is not part of this build: a config asking for it is refused.
"""

from __future__ import annotations

import torch

from difflet_amd.backends.rocm.component import RocmComponent


def wan_config(dit_config):
    """difflet_amd.dit.wan.WanConfig from a WanDiTConfig (WanTransformerConfig,
    difflet/models/wan/modeling_wan.py:114-160, plus the runtime shape; read by name)."""
    from difflet_amd.dit.wan import WanConfig

    c = dit_config
    if getattr(c, "cfg_parallel_enabled", False) or getattr(c, "context_parallel_enabled", False):
        raise NotImplementedError("CFG / context parallelism across GPUs is not part of this "
                                  "build: the rocm Wan component runs one GPU")
    if getattr(c, "qk_norm", "rms_norm_across_heads") != "rms_norm_across_heads":
        raise NotImplementedError("Wan's fused step normalises q/k across heads only")
    heads, hd = int(c.num_attention_heads), int(c.attention_head_dim)
    return WanConfig(hidden=heads * hd, heads=heads, head_dim=hd, ffn=int(c.ffn_dim),
                     n_blocks=int(c.num_layers), in_channels=int(c.in_channels),
                     out_channels=int(c.out_channels), text_dim=int(c.text_dim),
                     freq_dim=int(getattr(c, "freq_dim", 256)),
                     patch=tuple(getattr(c, "patch_size", (1, 2, 2))),
                     rope_max_seq_len=int(getattr(c, "rope_max_seq_len", 1024)))


class RocmWanTransformerApplication(RocmComponent):
    """One Wan expert on one MI355X. `kind` "bf16" (default) or "mx" (MXFP8 on the reference's
    Wan targets); `quantized_path` loads a quantized directory (difflet_amd.quant.checkpoint).
    `get`, when given, takes the module's parameter names (blocks.{i}.ffn.net_in.weight)."""

    def __init__(self, *, model_path=None, config, device=None, torch_compile: bool = False,
                 kind: str = "bf16", quantized_path=None, get=None):
        super().__init__(model_path=model_path if quantized_path is None else quantized_path,
                         config=config, device=device, torch_compile=torch_compile, get=get)
        if kind not in ("bf16", "mx"):
            raise ValueError(f"kind must be 'bf16' or 'mx', got {kind!r}")
        self.kind = kind
        self.quantized_path = quantized_path
        self.cfg = wan_config(config)

    def build_module(self):
        from difflet_amd.dit.wan import WanDiT, checkpoint_key

        if self.quantized_path is not None:
            return WanDiT.from_quantized_dir(self.cfg, self.quantized_path, device=self.device)
        if self._get is not None:
            get = self._get
        else:
            src = self.weight_source()
            get = lambda name: src(checkpoint_key(name))  # noqa: E731
        return WanDiT(self.cfg, get, device=self.device, kind=self.kind)

    def get_example_inputs(self) -> tuple:
        c = self.dit_config
        b, dt = int(getattr(c, "batch_size", 1)), self.dtype
        return (torch.zeros(b, int(c.in_channels), c.latent_frames, c.latent_height,
                            c.latent_width, dtype=dt),
                torch.zeros(b, dtype=dt),
                torch.zeros(b, int(c.text_seq_len), int(c.text_dim), dtype=dt))

    def forward(self, hidden_states, timestep, encoder_hidden_states):
        """[B, C, F, H, W] -> [B, C_out, F, H, W] in the model dtype."""
        dit = self._require_loaded()
        dev = self.device
        b = hidden_states.shape[0]
        t = timestep.reshape(-1)
        t = t.expand(b) if t.numel() == 1 else t
        outs = [dit.forward(hidden_states[i:i + 1].to(dev), t[i:i + 1].to(dev),
                            encoder_hidden_states[i:i + 1].to(dev)) for i in range(b)]
        return outs[0] if b == 1 else torch.cat(outs, dim=0)


__all__ = ["RocmWanTransformerApplication", "wan_config"]
