"""Wan 2.x text-to-video DiT denoise step on the gfx950 kernels: the fused form of
WanTransformer3DModel.forward (difflet/models/wan/modeling_wan.py:780-1068) with its block
(:671-763), attention (:472-668) and feed-forward (:377-430), bf16.

Per block, 13 launches: LayerNorm + modulation (fp32 vectors) -> [q|k|v] GEMM -> q/k RMSNorm
across heads + RoPE (stride-2 law) in place -> self-attention over all video tokens, output over
q -> output projection with gate * (x + b) + residual -> affine LayerNorm -> cross q GEMM and
text k/v GEMM -> q/k RMSNorm across heads -> cross-attention to the text -> output projection +
residual -> LayerNorm + modulation -> FFN in (GELU) -> FFN out with gate + residual.

HBM layout (batch 1, S video tokens, D = 5120, S_txt = 512): h [S, D] residual stream, n [S, D],
qkv [S, 3D] (self-attention; its first D columns also hold the cross-attention q), kv_txt
[S_txt, 2D], ff [S, 13824], txt [S_txt, D] embedded text; the modulation vectors of every block
as fp32 [blocks, 6, D] (the reference's scale_shift_table + timestep_proj, summed in fp32) and
the two gates as bf16.
"""

from __future__ import annotations

import math
from typing import Callable

import torch

from difflet_amd import _lib, kernels
from difflet_amd.dit.base import EPS
from difflet_amd.dit.linear import DeviceLinear, linear_group, run
from difflet_amd.dit.rope import wan_rope_tables


def patchify(latents: torch.Tensor, patch) -> torch.Tensor:
    """[C, F, H, W] -> [F/pt * H/ph * W/pw, C * pt * ph * pw], tokens frame-major, features in
    the (c, kt, kh, kw) order of a Conv3d weight: the patch embedding (kernel = stride = patch,
    modeling_wan.py:821-826) is then one linear."""
    ch, f, h, w = latents.shape
    pt, ph, pw = patch
    x = latents.reshape(ch, f // pt, pt, h // ph, ph, w // pw, pw)
    return x.permute(1, 3, 5, 0, 2, 4, 6).reshape(-1, ch * pt * ph * pw)


def unpatchify(y: torch.Tensor, grid, patch) -> torch.Tensor:
    """[F' * H' * W', pt * ph * pw * C] (features in (kt, kh, kw, c) order) -> [1, C, F, H, W], the
    reshape / permute of modeling_wan.py:1057-1059."""
    pt, ph, pw = patch
    y = y.reshape(*grid, pt, ph, pw, -1).permute(6, 0, 3, 1, 4, 2, 5)
    return y.reshape(1, -1, grid[0] * pt, grid[1] * ph, grid[2] * pw)


class WanConfig:
    def __init__(self, hidden=5120, heads=40, head_dim=128, ffn=13824, n_blocks=40,
                 in_channels=16, out_channels=16, text_dim=4096, freq_dim=256, patch=(1, 2, 2),
                 rope_max_seq_len=1024):
        self.hidden, self.heads, self.head_dim, self.ffn = hidden, heads, head_dim, ffn
        self.n_blocks, self.in_channels, self.out_channels = n_blocks, in_channels, out_channels
        self.text_dim, self.freq_dim, self.patch = text_dim, freq_dim, tuple(patch)
        self.rope_max_seq_len = rope_max_seq_len
        if heads * head_dim != hidden:
            raise ValueError("heads * head_dim must equal hidden")


#: difflet/models/wan/dit_config.py:126-139: the module's FFN attributes net_in / net_out are
#: diffusers' ffn.net.0.proj / ffn.net.2 in a checkpoint.
_MODULE_TO_CHECKPOINT = ((".ffn.net_in.", ".ffn.net.0.proj."), (".ffn.net_out.", ".ffn.net.2."))


def checkpoint_key(name: str) -> str:
    """The checkpoint key of the module parameter ``name``."""
    for module_part, ckpt_part in _MODULE_TO_CHECKPOINT:
        name = name.replace(module_part, ckpt_part)
    return name


class _Block:
    """kind "mx": the reference's MXFP8 Wan targets (difflet/quant/targets.py:259-263), the
    cross-attention's q/k/v and both FFN linears; self-attention and output projections bf16."""

    def __init__(self, get: Callable[[str], torch.Tensor], pre: str, kind: str = "bf16", q=None,
                 key: Callable[[str], str] = lambda n: n):
        W = lambda n: get(key(f"{pre}.{n}"))  # noqa: E731
        L = lambda k, *ns: linear_group(  # noqa: E731
            get, q, [key(f"{pre}.{n}.weight")[: -len(".weight")] for n in ns], k)
        self.qkv = L("bf16", "attn1.to_q", "attn1.to_k", "attn1.to_v")
        self.out1 = L("bf16", "attn1.to_out.0")
        self.q2 = L(kind, "attn2.to_q")
        self.kv2 = L(kind, "attn2.to_k", "attn2.to_v")
        self.out2 = L("bf16", "attn2.to_out.0")
        self.ffn_in = L(kind, "ffn.net_in")
        self.ffn_out = L(kind, "ffn.net_out")
        # an MXFP8 FFN: ffn_in's output rows in swizzle order, so its GELU -> MXFP8 epilogue
        # writes ffn_out's A operand
        self.ff_mx = (self.ffn_in.kind == "mx" and self.ffn_out.kind == "mx"
                      and self.ffn_in.n % 32 == 0)
        if self.ff_mx:
            self.ffn_in = self.ffn_in.rows_in_swizzle_order()
        bf = lambda n: W(n).to(torch.bfloat16).contiguous()  # noqa: E731
        self.nq1, self.nk1 = bf("attn1.norm_q.weight"), bf("attn1.norm_k.weight")
        self.nq2, self.nk2 = bf("attn2.norm_q.weight"), bf("attn2.norm_k.weight")
        f32 = lambda n: W(n).to(torch.float32).contiguous()  # noqa: E731
        self.norm2_w, self.norm2_b = f32("norm2.weight"), f32("norm2.bias")


class WanDiT:
    """The Wan transformer on the HIP kernels. `get(name)` returns a parameter by the reference
    module's name (blocks.{i}.attn1.to_q.weight, ...); `kind` "bf16" or "mx" (MXFP8 on the
    reference's Wan targets). `quantized` (a difflet_amd.quant.checkpoint.QuantizedCheckpoint)
    loads the linears it stores as fp8 from their codes and scales, `get` then taking checkpoint
    keys; WanDiT.from_quantized_dir builds the model from such a directory alone."""

    def __init__(self, cfg: WanConfig, get: Callable[[str], torch.Tensor],
                 device: str | torch.device = "cuda", kind: str = "bf16", quantized=None):
        key = lambda n: n  # noqa: E731
        if quantized is not None:
            kind = "fp8" if quantized.format == "fp8_rowwise" else "mx"
            key = checkpoint_key
        elif kind not in ("bf16", "mx"):
            raise ValueError(f"Wan runs kind 'bf16' or 'mx', got {kind!r}")
        self.cfg, self.kind = cfg, kind
        self.device = torch.device(device)
        G = lambda n: get(n).to(self.device)  # noqa: E731
        bf = lambda n: G(n).to(torch.bfloat16).contiguous()  # noqa: E731
        d = cfg.hidden
        pw = G("patch_embedding.weight")
        self.patch = DeviceLinear(pw.reshape(d, -1), G("patch_embedding.bias"))
        ce = "condition_embedder."
        self.t_w1, self.t_b1 = bf(ce + "time_embedder.linear_1.weight"), bf(ce + "time_embedder.linear_1.bias")
        self.t_w2, self.t_b2 = bf(ce + "time_embedder.linear_2.weight"), bf(ce + "time_embedder.linear_2.bias")
        self.tp_w, self.tp_b = bf(ce + "time_proj.weight"), bf(ce + "time_proj.bias")
        self.txt1 = DeviceLinear(G(ce + "text_embedder.linear_1.weight"), G(ce + "text_embedder.linear_1.bias"))
        self.txt2 = DeviceLinear(G(ce + "text_embedder.linear_2.weight"), G(ce + "text_embedder.linear_2.bias"))
        self.out_sst = G("scale_shift_table").to(torch.float32).reshape(2, d)
        self.proj_out = DeviceLinear(G("proj_out.weight"), G("proj_out.bias"))
        self.sst = torch.stack([G(f"blocks.{i}.scale_shift_table").to(torch.float32).reshape(6, d)
                                for i in range(cfg.n_blocks)])
        self.blocks = [_Block(G, f"blocks.{i}", kind, quantized, key) for i in range(cfg.n_blocks)]
        self.ones = torch.ones((1, d), dtype=torch.bfloat16, device=self.device)
        self._bufs: dict = {}
        self._rope: dict = {}
        self.probe = None

    def _timed(self, name: str):
        import contextlib

        return self.probe(name) if self.probe is not None else contextlib.nullcontext()

    def _buffers(self, s: int, st: int):
        key = (s, st)
        if key not in self._bufs:
            c, dev = self.cfg, self.device
            e = lambda *shape: torch.empty(shape, dtype=torch.bfloat16, device=dev)  # noqa: E731
            d = c.hidden
            bufs = {"h": e(s, d), "n": e(s, d), "qkv": e(s, 3 * d), "kv_txt": e(st, 2 * d),
                    "ff": e(s, c.ffn), "txt": e(st, d), "txt_tmp": e(st, d)}
            if self.kind == "mx" and d % 512 == 0:  # LayerNorm output straight to MXFP8
                bufs["nq"] = torch.empty((s, d), dtype=torch.float8_e4m3fn, device=dev)
                bufs["nsx"] = torch.empty((s, d // 32), dtype=torch.uint8, device=dev)
            if self.kind == "mx":  # the FFN hidden activation as MXFP8 from ffn_in's epilogue
                bufs["ffq"] = torch.empty((s, c.ffn), dtype=torch.float8_e4m3fn, device=dev)
                bufs["ffs"] = torch.empty((s, c.ffn // 32), dtype=torch.uint8, device=dev)
            self._bufs = {key: bufs}
        return self._bufs[key]

    def _ln(self, bufs, lin, mul, add, one_plus: bool = True):
        """LayerNorm (+ modulation or affine) of h into the A operand of linear `lin`: swizzled
        MXFP8 codes and scales in one pass for an MX linear, else bf16 into n."""
        if lin.kind == "mx" and "nsx" in bufs:
            out = (bufs["nq"], bufs["nsx"])
            kernels.layernorm_modulate_mx(bufs["h"], mul, add, eps=EPS, one_plus=one_plus, out=out)
            return out
        kernels.layernorm_modulate(bufs["h"], mul, add, eps=EPS, one_plus=one_plus, out=bufs["n"])
        return None

    def rope_tables(self, grid):
        key = tuple(grid)
        if key not in self._rope:
            self._rope = {key: wan_rope_tables(grid, self.cfg.head_dim, self.cfg.rope_max_seq_len,
                                               self.device)}
        return self._rope[key]

    def _gemm(self, name, problems, epilogue=0, act_col_start=0, kind="bf16"):
        with self._timed(name):
            run(problems, kind, epilogue, act_col_start)

    def _attention(self, qbuf, q_off, kbuf, k_off, vbuf, v_off):
        c = self.cfg
        view = lambda buf, off: buf.as_strided((1, c.heads, buf.shape[0], c.head_dim),  # noqa: E731
                                               (0, c.head_dim, buf.stride(0), 1),
                                               buf.storage_offset() + off)
        q = view(qbuf, q_off)
        with self._timed("attn.self" if kbuf is qbuf else "attn.cross"):
            kernels.attention(q, view(kbuf, k_off), view(vbuf, v_off),
                              scale=1.0 / math.sqrt(c.head_dim), out=q)

    def block(self, i: int, bufs, mods, gates, cos, sin):
        """mods fp32 [6, D] (shift, scale, gate, c_shift, c_scale, c_gate), gates bf16 [2, D]."""
        blk, c = self.blocks[i], self.cfg
        d = c.hidden
        h, n, qkv, kvt, ff, txt = (bufs[k] for k in ("h", "n", "qkv", "kv_txt", "ff", "txt"))
        sh, sc, _, c_sh, c_sc, _ = mods
        kernels.layernorm_modulate(h, sc, sh, eps=EPS, out=n)
        self._gemm("gemm.qkv", [blk.qkv.problem(n, qkv)], kind=blk.qkv.kind)
        kernels.qk_norm_rope(qkv, heads=c.heads, head_dim=c.head_dim, q_off=0, k_off=d,
                             wq=blk.nq1, wk=blk.nk1, eps=EPS, cos=cos, sin=sin, law=1, do_norm=2)
        self._attention(qkv, 0, qkv, d, qkv, 2 * d)
        self._gemm("gemm.out1", [blk.out1.problem(qkv[:, :d], h, gate=gates[0:1], residual=h)],
                   _lib.EPI_GATE_RESIDUAL, kind=blk.out1.kind)
        p = self._ln(bufs, blk.q2, blk.norm2_w, blk.norm2_b, one_plus=False)
        q2 = qkv[:, :d]
        self._gemm("gemm.q2", [blk.q2.problem(n, q2, prepared=p)], kind=blk.q2.kind)
        self._gemm("gemm.kv2", [blk.kv2.problem(txt, kvt)], kind=blk.kv2.kind)
        kernels.qk_norm_rope(qkv, heads=c.heads, head_dim=c.head_dim, q_off=0, k_off=-1,
                             wq=blk.nq2, wk=None, eps=EPS, cos=None, sin=None, do_norm=2)
        kernels.qk_norm_rope(kvt, heads=c.heads, head_dim=c.head_dim, q_off=0, k_off=-1,
                             wq=blk.nk2, wk=None, eps=EPS, cos=None, sin=None, do_norm=2)
        self._attention(qkv, 0, kvt, 0, kvt, d)
        self._gemm("gemm.out2", [blk.out2.problem(q2, h, gate=self.ones, residual=h)],
                   _lib.EPI_GATE_RESIDUAL, kind=blk.out2.kind)
        p = self._ln(bufs, blk.ffn_in, c_sc, c_sh)
        if blk.ff_mx and "ffq" in bufs:
            fq = (bufs["ffq"], bufs["ffs"])
            self._gemm("gemm.ffn_in", [blk.ffn_in.problem(n, fq[0], prepared=p, c_scale=fq[1])],
                       _lib.EPI_GELU_MX, kind="mx")
        else:
            self._gemm("gemm.ffn_in", [blk.ffn_in.problem(n, ff, prepared=p)], _lib.EPI_GELU,
                       kind=blk.ffn_in.kind)
            fq = None
        self._gemm("gemm.ffn_out", [blk.ffn_out.problem(ff, h, gate=gates[1:2], residual=h,
                                                        prepared=fq)],
                   _lib.EPI_GATE_RESIDUAL, kind=blk.ffn_out.kind)

    def condition(self, timestep, text, bufs):
        """(temb bf16 [1, D], timestep_proj bf16 [1, 6D]); the text projection into bufs['txt']."""
        dt = torch.bfloat16
        tp = kernels.timestep_embedding(timestep, self.cfg.freq_dim, flip_sin_to_cos=True,
                                        downscale_freq_shift=0.0, dtype=dt)
        temb = kernels.gemv(kernels.gemv(tp, self.t_w1, self.t_b1), self.t_w2, self.t_b2, act=1)
        tproj = kernels.gemv(temb, self.tp_w, self.tp_b, act=1)
        run([self.txt1.problem(text, bufs["txt_tmp"])], "bf16", _lib.EPI_GELU)
        run([self.txt2.problem(bufs["txt_tmp"], bufs["txt"])], "bf16")
        return temb, tproj

    def forward(self, latents, timestep, text):
        """latents [1, C, F, H, W], timestep [1] (0 .. 1000), text [1, S_txt, text_dim] ->
        [1, C_out, F, H, W] bf16."""
        if latents.shape[0] != 1:
            raise NotImplementedError("the fused Wan step runs batch 1 (one request per call)")
        c = self.cfg
        _, _, f, hh, ww = latents.shape
        pt, ph, pw = c.patch
        grid = (f // pt, hh // ph, ww // pw)
        s, st = grid[0] * grid[1] * grid[2], text.shape[1]
        bufs = self._buffers(s, st)
        cos, sin = self.rope_tables(grid)
        dt = torch.bfloat16
        self.patch(patchify(latents[0].to(dt), c.patch).contiguous(), out=bufs["h"])
        temb, tproj = self.condition(timestep.to(self.device).float(), text[0].to(dt).contiguous(), bufs)
        mods = self.sst + tproj.float().reshape(1, 6, -1)  # scale_shift_table + timestep_proj, fp32
        gates = mods[:, 2::3].to(dt).contiguous()           # gate, c_gate as bf16 [blocks, 2, D]
        for i in range(c.n_blocks):
            self.block(i, bufs, mods[i], gates[i], cos, sin)
        shift, scale = self.out_sst + temb.float()
        n = bufs["n"]
        kernels.layernorm_modulate(bufs["h"], scale, shift, eps=EPS, out=n)
        return unpatchify(self.proj_out(n), grid, c.patch)

    __call__ = forward

    @classmethod
    def from_quantized_dir(cls, cfg: WanConfig, path, device: str | torch.device = "cuda"
                           ) -> "WanDiT":
        """The model from a quantized directory alone (difflet_amd.quant.checkpoint), its keys
        diffusers' (checkpoint_key maps the module names)."""
        from difflet_amd.quant.checkpoint import QuantizedCheckpoint

        ckpt = QuantizedCheckpoint(path)
        return cls(cfg, ckpt.get, device=device, quantized=ckpt)


def wan_param_shapes(cfg: WanConfig) -> dict[str, tuple]:
    d, f = cfg.hidden, cfg.ffn
    out: dict[str, tuple] = {}

    def lin(n, o, i):
        out[f"{n}.weight"] = (o, i)
        out[f"{n}.bias"] = (o,)

    pt, ph, pw = cfg.patch
    out["patch_embedding.weight"] = (d, cfg.in_channels, pt, ph, pw)
    out["patch_embedding.bias"] = (d,)
    ce = "condition_embedder."
    lin(ce + "time_embedder.linear_1", d, cfg.freq_dim)
    lin(ce + "time_embedder.linear_2", d, d)
    lin(ce + "time_proj", 6 * d, d)
    lin(ce + "text_embedder.linear_1", d, cfg.text_dim)
    lin(ce + "text_embedder.linear_2", d, d)
    out["scale_shift_table"] = (1, 2, d)
    lin("proj_out", cfg.out_channels * pt * ph * pw, d)
    for b in range(cfg.n_blocks):
        p = f"blocks.{b}"
        out[f"{p}.scale_shift_table"] = (1, 6, d)
        for a in ("attn1", "attn2"):
            for n in ("to_q", "to_k", "to_v", "to_out.0"):
                lin(f"{p}.{a}.{n}", d, d)
            out[f"{p}.{a}.norm_q.weight"] = (d,)
            out[f"{p}.{a}.norm_k.weight"] = (d,)
        out[f"{p}.norm2.weight"] = (d,)
        out[f"{p}.norm2.bias"] = (d,)
        lin(f"{p}.ffn.net_in", f, d)
        lin(f"{p}.ffn.net_out", d, f)
    return out


def random_param_source(cfg: WanConfig, seed: int, device, std: float = 0.02):
    """Parameters drawn on the device on demand, N(0, std); norm weights ones, the LayerNorm
    bias zero; one generator per parameter seeded from (seed, name)."""
    import zlib

    shapes = wan_param_shapes(cfg)

    def get(name: str) -> torch.Tensor:
        shp = shapes[name]
        if name.endswith(("norm_q.weight", "norm_k.weight", "norm2.weight")):
            return torch.ones(shp, dtype=torch.bfloat16, device=device)
        if name.endswith("norm2.bias"):
            return torch.zeros(shp, dtype=torch.bfloat16, device=device)
        g = torch.Generator(device=device).manual_seed(seed * 1_000_003 + zlib.crc32(name.encode()))
        return (torch.randn(shp, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)

    return get
