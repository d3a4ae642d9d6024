"""FLUX.1 DiT denoise step on the gfx950 kernels: the fused, MI355X-first form of
NeuronFluxTransformer2DModel.forward (difflet/models/flux/modeling_flux.py:364-613).

This is the rocm backend's load-time module swap for FLUX (the reference's rule for a fusion of
one model on one backend, docs/design/gpu_backend.md:36-40): same weights (diffusers names),
same math, fewer HBM passes.

HBM layout, batch 1, S = S_txt + S_img tokens, D = hidden:
  h      [S, D] bf16     the residual stream, text rows first: the double blocks' two streams
                         are its two row ranges, so the double -> single concat is free.
  n      [S, D] bf16     LayerNorm + adaLN modulation output (the GEMM input).
  qkv    [S, 3D] bf16    double blocks: [q | k | v] per row from one GEMM per stream (text and
                         image grouped in one launch); q/k RMSNorm + RoPE in place; attention
                         reads q/k/v through strides and writes its output over q.
  big    [S, 7D] bf16    single blocks: [k | v | q | gelu(mlp)] from one GEMM (N = 7D, GELU
                         on the last 4D columns); attention output over q, so [attn | mlp] is
                         columns 2D..7D and proj_out is one K = 5D GEMM on that view with the
                         gate * (x + bias) + residual epilogue writing h in place.
  ff     [S, 4D] bf16    double blocks' MLP hidden (GELU fused into the up-projection).
  mod    [344 D] bf16    every block's adaLN vectors from one GEMV per step (temb is shared).
"""

from __future__ import annotations

from typing import Callable

import torch

from difflet_amd import _lib, kernels
from difflet_amd.dit.base import EPS, JointDiT
from difflet_amd.dit.linear import DeviceLinear, linear_group
from difflet_amd.dit.rope import flux_rope_tables


class FluxConfig:
    def __init__(self, hidden=3072, heads=24, head_dim=128, mlp_ratio=4, n_double=19,
                 n_single=38, in_channels=64, out_channels=64, txt_dim=4096, pooled_dim=768,
                 axes=(16, 56, 56), guidance=True):
        self.hidden, self.heads, self.head_dim = hidden, heads, head_dim
        self.mlp = hidden * mlp_ratio
        self.n_double, self.n_single = n_double, n_single
        self.in_channels, self.out_channels = in_channels, out_channels
        self.txt_dim, self.pooled_dim = txt_dim, pooled_dim
        self.axes, self.guidance = tuple(axes), guidance
        if heads * head_dim != hidden:
            raise ValueError("heads * head_dim must equal hidden")


class _Double:
    def __init__(self, get: Callable[[str], torch.Tensor], pre: str, cfg: FluxConfig, kind: str,
                 q=None):
        W = lambda n: get(f"{pre}.{n}")  # noqa: E731
        L = lambda *ns: linear_group(get, q, [f"{pre}.{n}" for n in ns], kind)  # noqa: E731
        a = "attn."
        self.qkv_img = L(a + "to_q", a + "to_k", a + "to_v")
        self.qkv_txt = L(a + "add_q_proj", a + "add_k_proj", a + "add_v_proj")
        self.out_img = L(a + "to_out.0")
        self.out_txt = L(a + "to_add_out")
        self.ff1_img = L("ff.net.0.proj")
        self.ff2_img = L("ff.net.2")
        self.ff1_txt = L("ff_context.net.0.proj")
        self.ff2_txt = L("ff_context.net.2")
        JointDiT._mx_mlp(self)
        bf = lambda n: W(n).to(torch.bfloat16).contiguous()  # noqa: E731
        self.nq, self.nk = bf(a + "norm_q.weight"), bf(a + "norm_k.weight")
        self.naq, self.nak = bf(a + "norm_added_q.weight"), bf(a + "norm_added_k.weight")


class _Single:
    def __init__(self, get: Callable[[str], torch.Tensor], pre: str, cfg: FluxConfig, kind: str,
                 q=None):
        W = lambda n: get(f"{pre}.{n}")  # noqa: E731
        a = "attn."
        # column order [k | v | q | mlp]: attention writes over q, leaving [attn | mlp] adjacent
        self.w1 = linear_group(get, q, [f"{pre}.{a}to_k", f"{pre}.{a}to_v", f"{pre}.{a}to_q",
                                  f"{pre}.proj_mlp"], kind)
        if q is not None and f"{pre}.proj_out.weight" not in q:
            # a checkpoint that splits proj_out stores proj_out_attn [D, D] and proj_out_mlp
            # [D, 4D]; the step runs them as the one K = 5D GEMM over [attn | mlp]
            self.w2 = linear_group(get, q, [f"{pre}.proj_out_attn", f"{pre}.proj_out_mlp"], kind,
                             along_k=True, bias_prefix=f"{pre}.proj_out")
        else:
            self.w2 = linear_group(get, q, [f"{pre}.proj_out"], kind)
        bf = lambda n: W(n).to(torch.bfloat16).contiguous()  # noqa: E731
        self.nq, self.nk = bf(a + "norm_q.weight"), bf(a + "norm_k.weight")


class FluxDiT(JointDiT):
    """The FLUX transformer on the HIP kernels. `get(name)` returns a parameter by its diffusers
    name (any dtype, on the target device); `kind` picks the block linears' format.

    `quantized` (a difflet_amd.quant.checkpoint.QuantizedCheckpoint) loads the block linears
    that a quantized checkpoint stores as fp8 from their codes and scales, with no quantization
    at load; `kind` then follows the checkpoint's format and the linears it keeps dense run in
    bf16. FluxDiT.from_quantized_dir builds the model from such a directory alone."""

    def __init__(self, cfg: FluxConfig, get: Callable[[str], torch.Tensor], kind: str = "bf16",
                 device: str | torch.device = "cuda", quantized=None):
        if quantized is not None:
            kind = "fp8" if quantized.format == "fp8_rowwise" else "mx"
        self.cfg, self.kind = cfg, kind
        self.device = torch.device(device)
        d = cfg.hidden
        G = lambda n: get(n).to(self.device)  # noqa: E731
        bf = lambda n: G(n).to(torch.bfloat16).contiguous()  # noqa: E731
        # embedders and the final layer stay bf16 (difflet/quant/targets.py:174-184)
        self.x_emb = DeviceLinear(G("x_embedder.weight"), G("x_embedder.bias"))
        self.ctx_emb = DeviceLinear(G("context_embedder.weight"), G("context_embedder.bias"))
        self.t_w1, self.t_b1 = bf("time_text_embed.timestep_embedder.linear_1.weight"), bf("time_text_embed.timestep_embedder.linear_1.bias")
        self.t_w2, self.t_b2 = bf("time_text_embed.timestep_embedder.linear_2.weight"), bf("time_text_embed.timestep_embedder.linear_2.bias")
        if cfg.guidance:
            self.g_w1, self.g_b1 = bf("time_text_embed.guidance_embedder.linear_1.weight"), bf("time_text_embed.guidance_embedder.linear_1.bias")
            self.g_w2, self.g_b2 = bf("time_text_embed.guidance_embedder.linear_2.weight"), bf("time_text_embed.guidance_embedder.linear_2.bias")
        self.p_w1, self.p_b1 = bf("time_text_embed.text_embedder.linear_1.weight"), bf("time_text_embed.text_embedder.linear_1.bias")
        self.p_w2, self.p_b2 = bf("time_text_embed.text_embedder.linear_2.weight"), bf("time_text_embed.text_embedder.linear_2.bias")
        self.proj_out = DeviceLinear(G("proj_out.weight"), G("proj_out.bias"))

        # every adaLN linear of the step in one [344 D, D] matrix: one GEMV per step
        mod_w, mod_b, self.mod_off = [], [], {}
        off = 0
        for i in range(cfg.n_double):
            for part in ("norm1", "norm1_context"):
                mod_w.append(bf(f"transformer_blocks.{i}.{part}.linear.weight"))
                mod_b.append(bf(f"transformer_blocks.{i}.{part}.linear.bias"))
                self.mod_off[("d", i, part)] = off
                off += 6 * d
        for i in range(cfg.n_single):
            mod_w.append(bf(f"single_transformer_blocks.{i}.norm.linear.weight"))
            mod_b.append(bf(f"single_transformer_blocks.{i}.norm.linear.bias"))
            self.mod_off[("s", i)] = off
            off += 3 * d
        mod_w.append(bf("norm_out.linear.weight"))
        mod_b.append(bf("norm_out.linear.bias"))
        self.mod_off["out"] = off
        off += 2 * d
        self.mod_w = torch.cat(mod_w, dim=0)
        self.mod_b = torch.cat(mod_b, dim=0)
        del mod_w, mod_b
        self.double = [_Double(G, f"transformer_blocks.{i}", cfg, kind, quantized)
                       for i in range(cfg.n_double)]
        self.single = [_Single(G, f"single_transformer_blocks.{i}", cfg, kind, quantized)
                       for i in range(cfg.n_single)]
        self._bufs: dict = {}
        self._rope: dict = {}
        #: per linear kind, whether the single block's q/k RMSNorm + RoPE runs in the W1 GEMM's
        #: epilogue (else as one launch after it)
        self.fuse_single_qk = {"bf16": True, "fp8": True, "mx": True}
        #: optional timing hook: probe(name) returns a context manager recording HIP events
        #: around a launch on the current stream (used by the benchmark, None otherwise)
        self.probe = None

    # -------------------------------------------------------------------------- helpers
    def _buffers(self, st: int, si: int):
        key = (st, si)
        if key not in self._bufs:
            s, d = st + si, self.cfg.hidden
            self._bufs = {key: self._new_buffers(s, {"big": (s, 7 * d),
                                                     "mod": (1, self.mod_w.shape[0])})}
        return self._bufs[key]

    def rope_tables(self, st: int, img_hw: tuple[int, int]):
        key = (st, tuple(img_hw))
        if key not in self._rope:
            self._rope = {key: flux_rope_tables(st, img_hw, self.cfg.axes, self.device)}
        return self._rope[key]

    # -------------------------------------------------------------------------- blocks
    def double_block(self, i: int, bufs, st: int, mod, cos, sin):
        self.joint_block(self.double[i], bufs, st,
                         self._mods(mod, self.mod_off[("d", i, "norm1")], 6),
                         self._mods(mod, self.mod_off[("d", i, "norm1_context")], 6),
                         cos, sin, "double")

    def single_block(self, i: int, bufs, mod, cos, sin):
        blk = self.single[i]
        c = self.cfg
        d = c.hidden
        h, n, big = bufs["h"], bufs["n"], bufs["big"]
        sh, sc, g = self._mods(mod, self.mod_off[("s", i)], 3)
        p = self._ln(bufs, slice(0, h.shape[0]), sc, sh, blk.w1.kind)
        # [k | v | q | mlp]: GELU on the MLP columns, q/k RMSNorm + RoPE in the same epilogue or
        # in one launch after it (self.fuse_single_qk)
        fuse = self.fuse_single_qk[blk.w1.kind]
        # per-token fp8: W1 stores the MLP pre-activation and W2's activation quantizer applies
        # the GELU (see JointDiT.fp8_gelu_at_quant)
        late = self._gelu_at_quant(blk.w2)
        self._gemm("gemm.single.w1",
                   [blk.w1.problem(n, big, prepared=p, norm_q=blk.nq, norm_k=blk.nk)],
                   blk.w1.kind, _lib.EPI_NONE if late else _lib.EPI_GELU, 0 if late else 3 * d,
                   qk=self._qk_epilogue(2 * d, 0, cos, sin) if fuse else None)
        if not fuse:
            kernels.qk_norm_rope(big, heads=c.heads, head_dim=c.head_dim, q_off=2 * d, k_off=0,
                                 wq=blk.nq, wk=blk.nk, eps=EPS, cos=cos, sin=sin, law=0)
        self._attn(big, 2 * d, 0, d)
        a2 = big[:, 2 * d:]
        self._gemm("gemm.single.w2",
                   [blk.w2.problem(a2, h, gate=g, residual=h,
                                   prepared=blk.w2.prep(a2, gelu_from=d) if late else None)],
                   blk.w2.kind, _lib.EPI_GATE_RESIDUAL)

    # -------------------------------------------------------------------------- step
    def embed(self, timestep, guidance, pooled):
        """temb [1, D] (difflet/layers/embeddings.py:247-281)."""
        dt = torch.bfloat16
        # the model casts timestep and guidance to its dtype and scales them there
        # (modeling_flux.py:453-456,477-479)
        timestep = timestep.to(dt) * 1000
        tp = kernels.timestep_embedding(timestep, 256, flip_sin_to_cos=True,
                                        downscale_freq_shift=0.0, dtype=dt)
        t = kernels.gemv(kernels.gemv(tp, self.t_w1, self.t_b1), self.t_w2, self.t_b2, act=1)
        if self.cfg.guidance:
            gp = kernels.timestep_embedding(guidance.to(dt) * 1000, 256, flip_sin_to_cos=True,
                                            downscale_freq_shift=0.0, dtype=dt)
            t = t + kernels.gemv(kernels.gemv(gp, self.g_w1, self.g_b1), self.g_w2, self.g_b2,
                                 act=1)
        p = kernels.gemv(kernels.gemv(pooled.to(dt), self.p_w1, self.p_b1), self.p_w2,
                         self.p_b2, act=1)
        return t + p

    def forward(self, latents, text, pooled, timestep, guidance, img_hw):
        """latents [1, S_img, in_ch], text [1, S_txt, txt_dim], pooled [1, pooled_dim],
        timestep / guidance [1] (timestep in [0, 1]) -> [1, S_img, out_ch] bf16. The RoPE
        table is FluxPosEmbed's over ids (0, 0, 0) for text and (0, i, j) for the img_hw grid."""
        cos, sin = self.rope_tables(text.shape[1], img_hw)
        return self.forward_rope(latents, text, pooled, timestep, guidance, cos, sin)

    def forward_rope(self, latents, text, pooled, timestep, guidance, cos, sin):
        """forward() with the RoPE table given: fp32 cos / sin [S_txt + S_img, head_dim] on the
        device, text rows first (the caller's ids, as the reference adapter builds them)."""
        if latents.shape[0] != 1:
            raise NotImplementedError("the fused FLUX step runs batch 1 (one request per call)")
        st, si = text.shape[1], latents.shape[1]
        shape = (st + si, self.cfg.head_dim)
        for name, t in (("cos", cos), ("sin", sin)):
            if (tuple(t.shape) != shape or t.dtype != torch.float32 or not t.is_contiguous()
                    or t.device != self.device):
                raise ValueError(f"forward_rope: {name} must be a contiguous fp32 {list(shape)} "
                                 f"on {self.device}")
        bufs = self._buffers(st, si)
        h = bufs["h"]
        dt = torch.bfloat16
        self.ctx_emb(text[0].to(dt).contiguous(), out=h[:st])
        self.x_emb(latents[0].to(dt).contiguous(), out=h[st:])
        temb = self.embed(timestep.to(self.device).float(), guidance.to(self.device).float(),
                          pooled.to(self.device))
        mod = kernels.gemv(temb, self.mod_w, self.mod_b, act=1, out=bufs["mod"])
        for i in range(self.cfg.n_double):
            self.double_block(i, bufs, st, mod, cos, sin)
        for i in range(self.cfg.n_single):
            self.single_block(i, bufs, mod, cos, sin)
        sc, sh = self._mods(mod, self.mod_off["out"], 2)  # AdaLN-Continuous: scale, shift
        n = bufs["n"]
        kernels.layernorm_modulate(h[st:], sc, sh, eps=EPS, out=n[st:])
        return self.proj_out(n[st:]).unsqueeze(0)

    __call__ = forward

    @classmethod
    def from_quantized_dir(cls, cfg: FluxConfig, path, device: str | torch.device = "cuda"
                           ) -> "FluxDiT":
        """The model from a quantized directory alone (difflet_amd.quant.checkpoint): fp8 block
        linears from their stored codes, every other tensor as stored."""
        from difflet_amd.quant.checkpoint import QuantizedCheckpoint

        ckpt = QuantizedCheckpoint(path)
        return cls(cfg, ckpt.get, device=device, quantized=ckpt)


def random_param_source(cfg: FluxConfig, seed: int, device, std: float = 0.02):
    """Parameters drawn on the device on demand, N(0, std) (RMSNorm weights ones), one
    generator per parameter seeded from (seed, name): the full model is built without a host
    copy. Not the oracle's draw (that one runs on the host); used where no CPU comparison of
    the same weights is made (the full-size step benchmark)."""
    import zlib

    shapes = flux_param_shapes(cfg)

    def get(name: str) -> torch.Tensor:
        shp = shapes[name]
        if ".norm_" in name and name.endswith(".weight") and len(shp) == 1:
            return torch.ones(shp, dtype=torch.bfloat16, device=device)
        g = torch.Generator(device=device).manual_seed(seed * 1_000_003 + zlib.crc32(name.encode()))
        return (torch.randn(shp, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)

    return get


def flux_param_shapes(cfg: FluxConfig) -> dict[str, tuple]:
    d, f, hd = cfg.hidden, cfg.mlp, cfg.head_dim
    out: dict[str, tuple] = {}

    def lin(n, o, i):
        out[f"{n}.weight"] = (o, i)
        out[f"{n}.bias"] = (o,)

    lin("x_embedder", d, cfg.in_channels)
    lin("context_embedder", d, cfg.txt_dim)
    for e, i in (("timestep_embedder", 256), ("guidance_embedder", 256),
                 ("text_embedder", cfg.pooled_dim)):
        lin(f"time_text_embed.{e}.linear_1", d, i)
        lin(f"time_text_embed.{e}.linear_2", d, d)
    lin("norm_out.linear", 2 * d, d)
    lin("proj_out", cfg.out_channels, d)
    for b in range(cfg.n_double):
        p = f"transformer_blocks.{b}"
        lin(f"{p}.norm1.linear", 6 * d, d)
        lin(f"{p}.norm1_context.linear", 6 * d, d)
        for n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_out.0",
                  "to_add_out"):
            lin(f"{p}.attn.{n}", d, d)
        for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
            out[f"{p}.attn.{n}.weight"] = (hd,)
        lin(f"{p}.ff.net.0.proj", f, d)
        lin(f"{p}.ff.net.2", d, f)
        lin(f"{p}.ff_context.net.0.proj", f, d)
        lin(f"{p}.ff_context.net.2", d, f)
    for b in range(cfg.n_single):
        p = f"single_transformer_blocks.{b}"
        lin(f"{p}.norm.linear", 3 * d, d)
        lin(f"{p}.proj_mlp", f, d)
        for n in ("to_q", "to_k", "to_v"):
            lin(f"{p}.attn.{n}", d, d)
        for n in ("norm_q", "norm_k"):
            out[f"{p}.attn.{n}.weight"] = (hd,)
        lin(f"{p}.proj_out", d, d + f)
    return out
