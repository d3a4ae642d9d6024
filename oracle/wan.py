"""Wan 2.x video DiT (text-to-video) restated in fp32 on the CPU, with seeded random weights.
Test infrastructure only (see oracle/__init__.py).

Follows difflet/models/wan/modeling_wan.py at tp = 1 without context / sequence / CFG
parallelism:
  WanRotaryPosEmbed      :209-296   (t / h / w axes of 44 / 42 / 42 dims for head_dim 128,
                                     float64 get_1d_rotary_pos_embed tables, repeat-interleaved,
                                     difflet/layers/embeddings.py:178-244)
  WanTimeTextEmbedding   :324-374   (sinusoid of 256 channels, cos first, shift 0; time embedder
                                     linear-SiLU-linear; time_proj of SiLU(temb) to 6 D;
                                     PixArt text projection linear-GELU(tanh)-linear)
  WanFeedForward         :377-430   (net_in, GELU-tanh, net_out)
  WanAttention           :472-668   (q/k/v, RMSNorm across heads in fp32 (:564-578 via
                                     difflet/backends/_torch_megatron/norm.py:35-45), rotary
                                     with the stride-2 law on self-attention only,
                                     difflet/backends/cpu/ops_impl/embeddings.py:6-14, scale
                                     1/sqrt(d), to_out)
  WanTransformerBlock    :671-763   (modulation = scale_shift_table + timestep_proj in fp32;
                                     fp32 LayerNorm + modulate; gate * attention + residual;
                                     affine fp32 LayerNorm + cross-attention + residual;
                                     LayerNorm + modulate + FFN, gate + residual)
  WanTransformer3DModel  :780-1068  (patch embedding Conv3d (1, 2, 2), blocks, norm_out with
                                     (shift, scale) = scale_shift_table + temb, proj_out,
                                     unpatchify)
FP32LayerNorm, Timesteps / TimestepEmbedding and PixArtAlphaTextProjection come from diffusers
0.38.0 (absent here); their published algorithms are the closed forms above (F.layer_norm in
fp32, the sinusoid, two linears around an activation). tests/test_oracle_wan.py pins condition,
final_layer and forward's composition by reductions to torch primitives and closed forms
(identity linears, distinct shift / scale rows), each with a planted mistake that fails it
(exact GELU in the text projection, a sin-first sinusoid, t cast to bf16 before the sinusoid,
shift and scale exchanged).

Weights: N(0, std) per block from torch.Generator(seed + block index) in spec order, rounded to
the model dtype; RMSNorm / LayerNorm weights ones, the LayerNorm bias zero.
"""

from __future__ import annotations

import dataclasses
import math

import torch

from oracle import ops
from oracle.flux import _draw


@dataclasses.dataclass(frozen=True)
class WanShape:
    hidden: int = 5120
    heads: int = 40
    head_dim: int = 128
    ffn: int = 13824
    n_blocks: int = 40
    in_channels: int = 16
    out_channels: int = 16
    text_dim: int = 4096
    freq_dim: int = 256
    patch: tuple = (1, 2, 2)
    rope_max_seq_len: int = 1024
    theta: float = 10000.0


WAN_14B = WanShape()
EMBED_SEED_OFFSET = 300_000


def block_params(shape: WanShape) -> list[tuple[str, tuple]]:
    d, f = shape.hidden, shape.ffn
    lin = lambda n, o, i: [(f"{n}.weight", (o, i)), (f"{n}.bias", (o,))]  # noqa: E731
    p = [("scale_shift_table", (1, 6, d))]
    for a in ("attn1", "attn2"):
        for n in ("to_q", "to_k", "to_v", "to_out.0"):
            p += lin(f"{a}.{n}", d, d)
        p += [(f"{a}.norm_q.weight", (d,)), (f"{a}.norm_k.weight", (d,))]
    p += [("norm2.weight", (d,)), ("norm2.bias", (d,))]
    p += lin("ffn.net_in", f, d)
    p += lin("ffn.net_out", d, f)
    return p


def embed_params(shape: WanShape) -> list[tuple[str, tuple]]:
    d = shape.hidden
    lin = lambda n, o, i: [(f"{n}.weight", (o, i)), (f"{n}.bias", (o,))]  # noqa: E731
    pt, ph, pw = shape.patch
    p = [("patch_embedding.weight", (d, shape.in_channels, pt, ph, pw)),
         ("patch_embedding.bias", (d,))]
    p += lin("condition_embedder.time_embedder.linear_1", d, shape.freq_dim)
    p += lin("condition_embedder.time_embedder.linear_2", d, d)
    p += lin("condition_embedder.time_proj", 6 * d, d)
    p += lin("condition_embedder.text_embedder.linear_1", d, shape.text_dim)
    p += lin("condition_embedder.text_embedder.linear_2", d, d)
    p += [("scale_shift_table", (1, 2, d))]
    p += lin("proj_out", shape.out_channels * pt * ph * pw, d)
    return p


def make_params(spec, seed: int, std: float = 0.02, dtype=torch.bfloat16) -> dict:
    g = torch.Generator().manual_seed(int(seed))
    out = {}
    for name, shp in spec:
        if name.endswith("norm_q.weight") or name.endswith("norm_k.weight") or name == "norm2.weight":
            t = torch.ones(shp)
        elif name == "norm2.bias":
            t = torch.zeros(shp)
        else:
            t = _draw(g, shp, std)
        out[name] = t.to(dtype).float()
    return out


def block_weights(shape: WanShape, seed: int, index: int, **kw) -> dict:
    return make_params(block_params(shape), seed + index, **kw)


def embed_weights(shape: WanShape, seed: int, **kw) -> dict:
    return make_params(embed_params(shape), seed + EMBED_SEED_OFFSET, **kw)


# ------------------------------------------------------------------------------------ RoPE
def rope_dims(head_dim: int) -> tuple[int, int, int]:
    hw = 2 * (head_dim // 6)
    return head_dim - 2 * hw, hw, hw


def _axis_table(dim: int, n: int, theta: float):
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64)[: dim // 2] / dim))
    ang = torch.outer(torch.arange(n, dtype=torch.float64), freqs)
    return ang.cos().repeat_interleave(2, dim=1).float(), ang.sin().repeat_interleave(2, dim=1).float()


def rope_tables(grid, shape: WanShape = WAN_14B):
    """(cos, sin) fp32 [F * H * W, head_dim] for the patch grid (F, H, W), frame-major."""
    f, h, w = grid
    tables = [_axis_table(dm, shape.rope_max_seq_len, shape.theta) for dm in rope_dims(shape.head_dim)]
    ff, yy, xx = torch.meshgrid(torch.arange(f), torch.arange(h), torch.arange(w), indexing="ij")
    idx = (ff.reshape(-1), yy.reshape(-1), xx.reshape(-1))
    cos = torch.cat([t[0][i] for t, i in zip(tables, idx)], dim=1)
    sin = torch.cat([t[1][i] for t, i in zip(tables, idx)], dim=1)
    return cos, sin


# ------------------------------------------------------------------------------------ block
def _attend(q, k, v, shape: WanShape):
    b, s, _ = q.shape
    h, d = shape.heads, shape.head_dim
    sh = lambda x: x.view(b, x.shape[1], h, d).transpose(1, 2).reshape(b * h, x.shape[1], d)  # noqa: E731
    o = ops.attention(sh(q), sh(k), sh(v), scale=1 / math.sqrt(d))
    return o.reshape(b, h, s, d).transpose(1, 2).reshape(b, s, h * d)


def block(w: dict, hidden, text, tproj, cos, sin, shape: WanShape, quant=None, act_dtype=None,
          store=None):
    """hidden [B, S, D], text [B, S_txt, D] (embedded), tproj [B, 6, D] -> hidden. `quant`
    ("mx") applies the MX law to the reference's Wan targets (difflet/quant/targets.py:259-263:
    the cross-attention's q/k/v and both FFN linears), the rest in fp32. `store` (a dtype)
    rounds every activation the device keeps in memory to it, and the two gates, which the
    device holds in that dtype; the shift / scale vectors stay fp32 as on the device."""
    from oracle.flux import qlinear

    L = ops.linear
    Q = qlinear(quant, act_dtype)
    R = ops.rounder(store)
    b, s, d = hidden.shape
    mods = w["scale_shift_table"] + tproj
    sh, sc, g, c_sh, c_sc, c_g = mods.chunk(6, dim=1)
    g, c_g = R(g), R(c_g)
    # self-attention
    nh = R(ops.layer_norm(hidden) * (1 + sc) + sh)
    q = ops.rms_norm_fp32(R(L(nh, w["attn1.to_q.weight"], w["attn1.to_q.bias"])), w["attn1.norm_q.weight"], 1e-6)
    k = ops.rms_norm_fp32(R(L(nh, w["attn1.to_k.weight"], w["attn1.to_k.bias"])), w["attn1.norm_k.weight"], 1e-6)
    v = R(L(nh, w["attn1.to_v.weight"], w["attn1.to_v.bias"]))
    rot = lambda x: R(ops.apply_rotary_emb(x.view(b, s, shape.heads, shape.head_dim),  # noqa: E731
                                           cos[None, :, None], sin[None, :, None]).reshape(b, s, d))
    q, k = rot(q), rot(k)
    o = L(R(_attend(q, k, v, shape)), w["attn1.to_out.0.weight"], w["attn1.to_out.0.bias"])
    hidden = R(hidden + o * g)
    # cross-attention to the text
    nh = R(torch.nn.functional.layer_norm(hidden, (d,), w["norm2.weight"], w["norm2.bias"], 1e-6))
    q = R(ops.rms_norm_fp32(R(Q(nh, w["attn2.to_q.weight"], w["attn2.to_q.bias"])), w["attn2.norm_q.weight"], 1e-6))
    k = R(ops.rms_norm_fp32(R(Q(text, w["attn2.to_k.weight"], w["attn2.to_k.bias"])), w["attn2.norm_k.weight"], 1e-6))
    v = R(Q(text, w["attn2.to_v.weight"], w["attn2.to_v.bias"]))
    hidden = R(hidden + L(R(_attend(q, k, v, shape)), w["attn2.to_out.0.weight"], w["attn2.to_out.0.bias"]))
    # feed-forward
    nh = R(ops.layer_norm(hidden) * (1 + c_sc) + c_sh)
    ff = Q(R(ops.gelu_tanh(Q(nh, w["ffn.net_in.weight"], w["ffn.net_in.bias"]))),
           w["ffn.net_out.weight"], w["ffn.net_out.bias"])
    return R(hidden + ff * c_g)


# ------------------------------------------------------------------------------------ model
def condition(ew: dict, timestep, text, model_dtype=torch.float32):
    """(temb [B, D], timestep_proj [B, 6, D], text [B, S_txt, D]); the time embedding is cast to
    the model dtype as the reference does (:356-361)."""
    L = ops.linear
    silu = torch.nn.functional.silu
    p = "condition_embedder."
    tp = ops.timestep_embedding(timestep.float(), 256, flip_sin_to_cos=True, downscale_freq_shift=0)
    tp = tp.to(model_dtype).float()
    temb = L(silu(L(tp, ew[p + "time_embedder.linear_1.weight"], ew[p + "time_embedder.linear_1.bias"])),
             ew[p + "time_embedder.linear_2.weight"], ew[p + "time_embedder.linear_2.bias"])
    temb = temb.to(model_dtype).float()
    tproj = L(silu(temb), ew[p + "time_proj.weight"], ew[p + "time_proj.bias"]).to(model_dtype).float()
    txt = L(ops.gelu_tanh(L(text, ew[p + "text_embedder.linear_1.weight"], ew[p + "text_embedder.linear_1.bias"])),
            ew[p + "text_embedder.linear_2.weight"], ew[p + "text_embedder.linear_2.bias"])
    return temb, tproj.unflatten(1, (6, -1)), txt


def forward(shape: WanShape, seed: int, latents, timestep, text, weights=None,
            dtype=torch.bfloat16, model_dtype=torch.float32):
    """latents [B, C, F, H, W], timestep [B] (0 .. 1000), text [B, S_txt, text_dim] ->
    [B, C_out, F, H, W]. Blocks are drawn one at a time unless `weights` = (embed, [block...])."""
    ew = weights[0] if weights else embed_weights(shape, seed, dtype=dtype)
    b, _, f, h, w = latents.shape
    pt, ph, pw = shape.patch
    grid = (f // pt, h // ph, w // pw)
    x = torch.nn.functional.conv3d(latents, ew["patch_embedding.weight"], ew["patch_embedding.bias"],
                                   stride=shape.patch)
    hidden = x.flatten(2).transpose(1, 2)
    temb, tproj, txt = condition(ew, timestep, text, model_dtype)
    cos, sin = rope_tables(grid, shape)
    for i in range(shape.n_blocks):
        wb = weights[1][i] if weights else block_weights(shape, seed, i, dtype=dtype)
        hidden = block(wb, hidden, txt, tproj, cos, sin, shape)
    out = final_layer(ew, hidden, temb)
    out = out.reshape(b, *grid, pt, ph, pw, -1).permute(0, 7, 1, 4, 2, 5, 3, 6)
    return out.flatten(6, 7).flatten(4, 5).flatten(2, 3)


def final_layer(ew: dict, hidden, temb):
    """norm_out + proj_out (:1031-1044): (shift, scale) = scale_shift_table + temb, in that
    chunk order; fp32 LayerNorm without affine, x (1 + scale) + shift, then proj_out.
    hidden [B, S, D], temb [B, D] -> [B, S, out_ch * prod(patch)]."""
    shift, scale = (ew["scale_shift_table"] + temb[:, None]).chunk(2, dim=1)
    hidden = ops.layer_norm(hidden) * (1 + scale) + shift
    return ops.linear(hidden, ew["proj_out.weight"], ew["proj_out.bias"])


def synthetic_inputs(shape: WanShape, seed: int, latent_fhw, txt_len, batch: int = 1):
    """latents [B, C, F, H, W] and text [B, txt_len, text_dim] ~ N(0, 1); timestep ~ U[0, 1000)."""
    g = torch.Generator().manual_seed(int(seed))
    f, h, w = latent_fhw
    latents = torch.randn(batch, shape.in_channels, f, h, w, generator=g)
    text = torch.randn(batch, txt_len, shape.text_dim, generator=g)
    t = torch.rand(batch, generator=g) * 1000.0
    return {"latents": latents, "text": text, "timestep": t}
