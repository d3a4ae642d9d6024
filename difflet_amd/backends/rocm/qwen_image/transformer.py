"""The Qwen-Image DiT as a rocm GPU component, replacing difflet/backends/cuda/qwen_image/
transformer.py:31-121 (the load-time module swap of docs/design/gpu_backend.md:36-40 for
Qwen-Image).

`RocmQwenImageTransformerApplication` builds the fused step (difflet_amd.dit.qwen.
QwenImageDiT) from a diffusers `transformer/` directory and runs it with the CUDA component's
forward signature: (hidden_states, timestep, encoder_hidden_states,
encoder_hidden_states_mask=None, guidance=None), timestep being t / 1000 as QwenImagePipeline
passes it. A right-padded prompt's mask is handled as the CUDA component handles it
(apply_text_mask with trim_text_padding, modeling_qwen_image.py:555-576,695-722): the text is
cut after its last valid row, which gives the masked output for the image tokens; a mask with
holes inside the prompt is refused. The packed latent grid comes from the config
(packed_height x packed_width, modeling_qwen_image.py:710-716) or, for another sequence
length, from a square grid.
"""

from __future__ import annotations

import math
import os

import torch

from difflet_amd.backends.rocm.component import RocmComponent

# the reference's prefix of the DiT's parameters inside its trace module; the checkpoint's own
# keys are bare, which is how the fused step reads them
CHECKPOINT_PREFIX = "transformer."
WARMUP_VALID_TEXT_TOKENS = 37


def qwen_config(dit_config):
    """difflet_amd.dit.qwen.QwenConfig from a QwenImageDiTConfig (difflet/models/qwen_image/
    dit_config.py:29-52; read by attribute name)."""
    from difflet_amd.dit.qwen import QwenConfig

    c = dit_config
    heads, hd = int(c.num_attention_heads), int(c.attention_head_dim)
    if getattr(c, "guidance_embeds", False):
        raise NotImplementedError("the fused Qwen-Image step has no guidance embedder")
    if getattr(c, "zero_cond_t", False) or getattr(c, "use_layer3d_rope", False):
        raise NotImplementedError("zero_cond_t / use_layer3d_rope are not part of the fused step")
    return QwenConfig(hidden=heads * hd, heads=heads, head_dim=hd, mlp=4 * heads * hd,
                      n_blocks=int(c.num_layers), in_channels=int(c.in_channels),
                      out_channels=int(c.out_channels), txt_dim=int(c.joint_attention_dim),
                      axes=tuple(c.axes_dims_rope))


def trim_text_padding(encoder_hidden_states: torch.Tensor, mask: torch.Tensor | None):
    """(text, valid rows) of one request: the prompt cut after its last valid row
    (modeling_qwen_image.py:555-576). A mask with no valid row, or with a padded row before
    the last valid one, is refused (the fused step bounds the text keys by a prefix)."""
    if mask is None:
        return encoder_hidden_states, encoder_hidden_states.shape[1]
    mask = mask.to(torch.bool).reshape(-1).cpu()
    if not bool(mask.any()):
        raise ValueError("encoder_hidden_states_mask has no valid text token")
    length = int(torch.nonzero(mask).max()) + 1
    if not bool(mask[:length].all()):
        raise NotImplementedError("a text mask with padded rows inside the prompt is not "
                                  "supported by the fused Qwen-Image step (right padding only)")
    return encoder_hidden_states[:, :length], length


class RocmQwenImageTransformerApplication(RocmComponent):
    """Qwen-Image's DiT on one MI355X. `kind` "mx" (default: MXFP8 on QWEN_IMAGE_TARGETS) or
    "bf16"; `quantized_path` loads a quantized directory (difflet_amd.quant.checkpoint)."""

    def __init__(self, *, model_path=None, config, device=None, torch_compile: bool = False,
                 kind: str = "mx", quantized_path=None, get=None):
        super().__init__(model_path=model_path if quantized_path is None else quantized_path,
                         config=config, device=device, torch_compile=torch_compile, get=get)
        if kind not in ("bf16", "mx"):
            raise ValueError(f"kind must be 'bf16' or 'mx', got {kind!r}")
        self.kind = kind
        self.quantized_path = quantized_path
        self.cfg = qwen_config(config)

    def build_module(self):
        from difflet_amd.dit.qwen import QwenImageDiT

        if self.quantized_path is not None:
            return QwenImageDiT.from_quantized_dir(self.cfg, self.quantized_path,
                                                   device=self.device)
        return QwenImageDiT(self.cfg, self.weight_source(), kind=self.kind, device=self.device)

    def packed_hw(self, image_seq_len: int) -> tuple[int, int]:
        c = self.dit_config
        ph, pw = getattr(c, "packed_height", None), getattr(c, "packed_width", None)
        if ph is not None and pw is not None and int(ph) * int(pw) == image_seq_len:
            return int(ph), int(pw)
        r = math.isqrt(image_seq_len)
        if r * r != image_seq_len:
            raise ValueError(f"{image_seq_len} image tokens are neither the configured "
                             f"{ph} x {pw} grid nor a square one")
        return r, r

    def get_example_inputs(self) -> tuple:
        c = self.dit_config
        b, dt = int(getattr(c, "batch_size", 1)), self.dtype
        mask = torch.zeros(b, int(c.text_seq_len), dtype=torch.bool)
        mask[:, : min(WARMUP_VALID_TEXT_TOKENS, int(c.text_seq_len))] = True
        return (torch.zeros(b, int(c.image_seq_len), int(c.in_channels), dtype=dt),
                torch.zeros(b, dtype=dt),
                torch.zeros(b, int(c.text_seq_len), int(c.joint_attention_dim), dtype=dt),
                mask, None)

    def forward(self, hidden_states, timestep, encoder_hidden_states,
                encoder_hidden_states_mask=None, guidance=None, *, text_valid_len=None):
        """[B, S_img, in_ch] -> [B, S_img, out_ch] in the model dtype, one request per launch
        sequence. `text_valid_len` (an int per request, the neuron path's form of the mask)
        may replace the mask."""
        dit = self._require_loaded()
        del guidance  # no guidance embedder (qwen_config refuses one)
        dev = self.device
        b = hidden_states.shape[0]
        hw = self.packed_hw(int(hidden_states.shape[1]))
        t = timestep.reshape(-1)
        t = t.expand(b) if t.numel() == 1 else t
        outs = []
        for i in range(b):
            text = encoder_hidden_states[i:i + 1]
            if encoder_hidden_states_mask is not None:
                text, _ = trim_text_padding(text, encoder_hidden_states_mask[i])
            valid = None
            if text_valid_len is not None:
                tv = text_valid_len.reshape(-1) if torch.is_tensor(text_valid_len) \
                    else torch.tensor([int(text_valid_len)])
                valid = int(tv[i] if tv.numel() > 1 else tv[0])
            outs.append(dit.forward(hidden_states[i:i + 1].to(dev), text.to(dev),
                                    t[i:i + 1].to(dev), hw, text_valid_len=valid))
        return outs[0] if b == 1 else torch.cat(outs, dim=0)


def transformer_dir(model_path: str) -> str:
    return os.path.join(model_path, "transformer")


__all__ = ["CHECKPOINT_PREFIX", "RocmQwenImageTransformerApplication", "WARMUP_VALID_TEXT_TOKENS",
           "qwen_config", "transformer_dir", "trim_text_padding"]
