"""Qwen-Image MMDiT denoise step on the gfx950 kernels: the fused form of diffusers'
QwenImageTransformer2DModel as the reference runs it (difflet/models/qwen_image/
modeling_qwen_image.py:579-770) with its joint block (difflet/models/qwen_image/
modeling_qwen.py:107-285) and attention processor (modeling_qwen_image.py:317-491).

The 60 joint blocks run the shared joint-block sequence (difflet_amd/dit/base.py). With
kind "mx" the MXFP8 targets (QWEN_IMAGE_TARGETS, difflet/quant/targets.py:117-121: q/k/v, the
added q/k/v, both MLPs) run the MXFP8 GEMM, their activations quantized per call with the MX
block law; the output projections, embedders, modulation and final layer stay bf16.

HBM layout (batch 1, S = 256 text + 6889 image tokens, D = 3072): h [S, D] text rows first,
n [S, D], qkv [S, 3D], ff [S, 12288], mod [722 D] (every block's img_mod and txt_mod vectors and
the final AdaLN-Continuous pair from one GEMV per step).
"""

from __future__ import annotations

from typing import Callable

import torch

from difflet_amd import kernels
from difflet_amd.dit.base import EPS, JointDiT
from difflet_amd.dit.linear import DeviceLinear, linear_group
from difflet_amd.dit.rope import qwen_rope_tables


class QwenConfig:
    def __init__(self, hidden=3072, heads=24, head_dim=128, mlp=12288, n_blocks=60,
                 in_channels=64, out_channels=64, txt_dim=3584, axes=(16, 56, 56)):
        self.hidden, self.heads, self.head_dim, self.mlp = hidden, heads, head_dim, mlp
        self.n_blocks, self.in_channels, self.out_channels = n_blocks, in_channels, out_channels
        self.txt_dim, self.axes = txt_dim, tuple(axes)
        if heads * head_dim != hidden:
            raise ValueError("heads * head_dim must equal hidden")


class _Block:
    def __init__(self, get: Callable[[str], torch.Tensor], pre: str, kind: str, q=None):
        W = lambda n: get(f"{pre}.{n}")  # noqa: E731
        L = lambda *ns, k=kind: linear_group(get, q, [f"{pre}.{n}" for n in ns], k)  # noqa: E731
        a = "attn."
        self.qkv_img = L(a + "to_q", a + "to_k", a + "to_v")
        self.qkv_txt = L(a + "add_q_proj", a + "add_k_proj", a + "add_v_proj")
        # the output projections are not MXFP8 targets
        self.out_img = L(a + "to_out.0", k="bf16")
        self.out_txt = L(a + "to_add_out", k="bf16")
        self.ff1_img = L("img_mlp.net.0.proj")
        self.ff2_img = L("img_mlp.net.2")
        self.ff1_txt = L("txt_mlp.net.0.proj")
        self.ff2_txt = L("txt_mlp.net.2")
        JointDiT._mx_mlp(self)
        bf = lambda n: W(n).to(torch.bfloat16).contiguous()  # noqa: E731
        self.nq, self.nk = bf(a + "norm_q.weight"), bf(a + "norm_k.weight")
        self.naq, self.nak = bf(a + "norm_added_q.weight"), bf(a + "norm_added_k.weight")


class QwenImageDiT(JointDiT):
    """The Qwen-Image transformer on the HIP kernels. `get(name)` returns a parameter by its
    diffusers name; `kind` is "bf16" or "mx" (MXFP8 on the targeted block linears).

    `quantized` (a difflet_amd.quant.checkpoint.QuantizedCheckpoint) loads the block linears a
    quantized checkpoint stores as fp8 from their codes and scales, with no quantization at
    load (`kind` then follows its format); QwenImageDiT.from_quantized_dir builds the model
    from such a directory alone."""

    def __init__(self, cfg: QwenConfig, get: Callable[[str], torch.Tensor], kind: str = "mx",
                 device: str | torch.device = "cuda", quantized=None):
        if quantized is not None:
            kind = "fp8" if quantized.format == "fp8_rowwise" else "mx"
        elif kind not in ("bf16", "mx"):
            raise ValueError(f"Qwen-Image runs kind 'bf16' or 'mx', got {kind!r}")
        self.cfg, self.kind = cfg, kind
        self.device = torch.device(device)
        d = cfg.hidden
        G = lambda n: get(n).to(self.device)  # noqa: E731
        bf = lambda n: G(n).to(torch.bfloat16).contiguous()  # noqa: E731
        self.img_in = DeviceLinear(G("img_in.weight"), G("img_in.bias"))
        self.txt_norm = bf("txt_norm.weight")
        self.txt_in = DeviceLinear(G("txt_in.weight"), G("txt_in.bias"))
        te = "time_text_embed.timestep_embedder."
        self.t_w1, self.t_b1 = bf(te + "linear_1.weight"), bf(te + "linear_1.bias")
        self.t_w2, self.t_b2 = bf(te + "linear_2.weight"), bf(te + "linear_2.bias")
        self.proj_out = DeviceLinear(G("proj_out.weight"), G("proj_out.bias"))
        mod_w, mod_b, self.mod_off = [], [], {}
        off = 0
        for i in range(cfg.n_blocks):
            for part in ("img_mod", "txt_mod"):
                mod_w.append(bf(f"transformer_blocks.{i}.{part}.1.weight"))
                mod_b.append(bf(f"transformer_blocks.{i}.{part}.1.bias"))
                self.mod_off[(i, part)] = off
                off += 6 * d
        mod_w.append(bf("norm_out.linear.weight"))
        mod_b.append(bf("norm_out.linear.bias"))
        self.mod_off["out"] = off
        self.mod_w = torch.cat(mod_w, dim=0)
        self.mod_b = torch.cat(mod_b, dim=0)
        del mod_w, mod_b
        self.blocks = [_Block(G, f"transformer_blocks.{i}", kind, quantized)
                       for i in range(cfg.n_blocks)]
        self._bufs: dict = {}
        self._rope: dict = {}
        self.probe = None

    def _buffers(self, st: int, si: int):
        key = (st, si)
        if key not in self._bufs:
            self._bufs = {key: self._new_buffers(st + si, {"mod": (1, self.mod_w.shape[0])})}
        return self._bufs[key]

    def rope_tables(self, st: int, img_hw: tuple[int, int]):
        key = (st, tuple(img_hw))
        if key not in self._rope:
            self._rope = {key: qwen_rope_tables(st, img_hw, self.cfg.axes, self.device)}
        return self._rope[key]

    def block(self, i: int, bufs, st: int, mod, cos, sin):
        self.joint_block(self.blocks[i], bufs, st, self._mods(mod, self.mod_off[(i, "img_mod")], 6),
                         self._mods(mod, self.mod_off[(i, "txt_mod")], 6), cos, sin, "joint")

    def embed(self, timestep):
        """temb [1, D]: the model casts t / 1000 to bf16, the sinusoid scales it by 1000."""
        t = timestep.to(torch.bfloat16).float() * 1000.0
        tp = kernels.timestep_embedding(t, 256, flip_sin_to_cos=True, downscale_freq_shift=0.0,
                                        dtype=torch.bfloat16)
        return kernels.gemv(kernels.gemv(tp, self.t_w1, self.t_b1), self.t_w2, self.t_b2, act=1)

    def forward(self, latents, text, timestep, img_hw, text_valid_len=None):
        """latents [1, h*w, in_ch] (packed 2x2 patches), text [1, S_txt, txt_dim], timestep t/1000
        [1] -> [1, h*w, out_ch] bf16.

        ``text_valid_len`` (int, or an int tensor of one element) marks a right-padded prompt:
        only its first rows are keys. The reference masks the padding keys in every block
        (keys [image | text] bounded at S_img + valid, modeling_qwen_image.py:493-552,
        738-739); for one request the padded rows are then keys to nobody and their own
        outputs are dropped, so the step runs the prompt cut to its valid rows, which gives
        the same image output (the reference's trim_text_padding, :555-576) on a shorter
        joint sequence."""
        if latents.shape[0] != 1:
            raise NotImplementedError("the fused Qwen-Image step runs batch 1 (one request per call)")
        if text_valid_len is not None:
            valid = int(text_valid_len.reshape(-1)[0]) if torch.is_tensor(text_valid_len) \
                else int(text_valid_len)
            if torch.is_tensor(text_valid_len) and text_valid_len.numel() != 1:
                raise NotImplementedError("the fused Qwen-Image step takes one text_valid_len")
            if not 0 <= valid <= text.shape[1]:
                raise ValueError(f"text_valid_len {valid} outside [0, {text.shape[1]}]")
            text = text[:, :valid]
        st, si = text.shape[1], latents.shape[1]
        bufs = self._buffers(st, si)
        cos, sin = self.rope_tables(st, img_hw)
        h, n = bufs["h"], bufs["n"]
        dt = torch.bfloat16
        tn = kernels.rms_norm(text[0].to(dt).contiguous(), self.txt_norm, EPS)
        self.txt_in(tn, out=h[:st])
        self.img_in(latents[0].to(dt).contiguous(), out=h[st:])
        temb = self.embed(timestep.to(self.device).float())
        mod = kernels.gemv(temb, self.mod_w, self.mod_b, act=1, out=bufs["mod"])
        for i in range(self.cfg.n_blocks):
            self.block(i, bufs, st, mod, cos, sin)
        sc, sh = self._mods(mod, self.mod_off["out"], 2)  # AdaLN-Continuous: scale, shift
        kernels.layernorm_modulate(h[st:], sc, sh, eps=EPS, out=n[st:])
        return self.proj_out(n[st:]).unsqueeze(0)

    __call__ = forward

    @classmethod
    def from_quantized_dir(cls, cfg: QwenConfig, path, device: str | torch.device = "cuda"
                           ) -> "QwenImageDiT":
        """The model from a quantized directory alone (difflet_amd.quant.checkpoint)."""
        from difflet_amd.quant.checkpoint import QuantizedCheckpoint

        ckpt = QuantizedCheckpoint(path)
        return cls(cfg, ckpt.get, device=device, quantized=ckpt)


def qwen_param_shapes(cfg: QwenConfig) -> dict[str, tuple]:
    d, f, hd = cfg.hidden, cfg.mlp, cfg.head_dim
    out: dict[str, tuple] = {}

    def lin(n, o, i):
        out[f"{n}.weight"] = (o, i)
        out[f"{n}.bias"] = (o,)

    lin("img_in", d, cfg.in_channels)
    out["txt_norm.weight"] = (cfg.txt_dim,)
    lin("txt_in", d, cfg.txt_dim)
    lin("time_text_embed.timestep_embedder.linear_1", d, 256)
    lin("time_text_embed.timestep_embedder.linear_2", d, d)
    lin("norm_out.linear", 2 * d, d)
    lin("proj_out", cfg.out_channels, d)
    for b in range(cfg.n_blocks):
        p = f"transformer_blocks.{b}"
        lin(f"{p}.img_mod.1", 6 * d, d)
        lin(f"{p}.txt_mod.1", 6 * d, d)
        for n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_out.0",
                  "to_add_out"):
            lin(f"{p}.attn.{n}", d, d)
        for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
            out[f"{p}.attn.{n}.weight"] = (hd,)
        for s in ("img_mlp", "txt_mlp"):
            lin(f"{p}.{s}.net.0.proj", f, d)
            lin(f"{p}.{s}.net.2", d, f)
    return out


def random_param_source(cfg: QwenConfig, seed: int, device, std: float = 0.02):
    """Parameters drawn on the device on demand, N(0, std) (RMSNorm weights ones), one generator
    per parameter seeded from (seed, name); used by the full-size benchmark."""
    import zlib

    shapes = qwen_param_shapes(cfg)

    def get(name: str) -> torch.Tensor:
        shp = shapes[name]
        if name.endswith(".weight") and len(shp) == 1 and (".norm_" in name or name.startswith("txt_norm.")):
            return torch.ones(shp, dtype=torch.bfloat16, device=device)
        g = torch.Generator(device=device).manual_seed(seed * 1_000_003 + zlib.crc32(name.encode()))
        return (torch.randn(shp, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)

    return get
