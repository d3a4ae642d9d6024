"""Qwen-Image MMDiT restated in fp32 on the CPU, with seeded random weights. Test
infrastructure only (see oracle/__init__.py).

Block: difflet/models/qwen_image/modeling_qwen.py:107-285 (QwenImageSPTransformerBlock at
sp = tp = 1) with the attention of difflet/models/qwen_image/modeling_qwen_image.py:317-491
(_QwenImageTrainiumAttnProcessor, unmasked joint path :442-466): per-stream q/k/v, per-head
RMSNorm, real-valued RoPE (:58-67, the interleaved-pair law), joint [txt | img] attention with
scale 1/sqrt(d), split at the text length, to_out.0 / to_add_out, gate * out + residual, then
per-stream LayerNorm + modulation + GELU-tanh MLP.

Model level: diffusers' QwenImageTransformer2DModel (diffusers 0.38.0, pyproject.toml:34), which
the reference builds at modeling_qwen_image.py:652-667 and which is absent here. Restated from
its published algorithm: img_in, txt_norm (RMSNorm) + txt_in, the timestep projection
(sinusoid of 256 channels, flip_sin_to_cos, shift 0, scale 1000, then linear-SiLU-linear),
AdaLN-Continuous norm_out (scale first) and proj_out; the 3-axis RoPE table of QwenEmbedRope
with scale_rope (image height / width positions centred on zero, text positions from
max(h // 2, w // 2)), angles computed in fp32. No fixture of the reference covers these
model-level pieces; tests/test_oracle_qwen.py pins time_embed, embed_text, final_layer and
forward's composition by reductions to torch primitives and closed forms (identity linears,
distinct scale / shift vectors), each with a planted mistake that fails it (sin-first
sinusoid, a cast after the 1000 scale, LayerNorm for txt_norm, shift-first AdaLN-Continuous).
Parity unpinned: the RMSNorm rounding order of diffusers in bf16 (normalise in fp32, round to
the weight dtype, multiply by the weight; the oracle computes the fp32 law) and the
pos_embed table beyond its closed form (test_rope_table_closed_form restates the published
rule; the device and this oracle consume the same table).

MXFP8 (config: every targeted linear, QWEN_IMAGE_TARGETS of difflet/quant/targets.py:117-121):
q/k/v, the added q/k/v and both MLPs take FakeQuantMXLinear's law (difflet/quant/
fake_linear.py:56-61: both operands through the MX block law, product in fp32); the output
projections and the modulation linears stay full precision.
"""

from __future__ import annotations

import dataclasses
import math

import torch

from oracle import ops
from oracle.flux import _draw, gelu_input_rounder, qlinear


@dataclasses.dataclass(frozen=True)
class QwenShape:
    hidden: int = 3072
    heads: int = 24
    head_dim: int = 128
    mlp: int = 12288
    n_blocks: int = 60
    in_channels: int = 64
    out_channels: int = 64  # patch 2 x 2 x 16 latent channels
    txt_dim: int = 3584
    axes: tuple = (16, 56, 56)
    theta: int = 10000


QWEN_IMAGE = QwenShape()
EMBED_SEED_OFFSET = 200_000

#: the block linears MXFP8 quantizes (QWEN_IMAGE_TARGETS), by parameter prefix
MX_TARGETS = ("attn.to_q", "attn.to_k", "attn.to_v", "attn.add_q_proj", "attn.add_k_proj",
              "attn.add_v_proj", "img_mlp.net.0.proj", "img_mlp.net.2", "txt_mlp.net.0.proj",
              "txt_mlp.net.2")


def block_params(shape: QwenShape) -> list[tuple[str, tuple]]:
    d, f, hd = shape.hidden, shape.mlp, shape.head_dim
    lin = lambda n, o, i: [(f"{n}.weight", (o, i)), (f"{n}.bias", (o,))]  # noqa: E731
    p = []
    p += lin("img_mod.1", 6 * d, d)
    p += lin("txt_mod.1", 6 * d, d)
    for n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj"):
        p += lin(f"attn.{n}", d, d)
    p += lin("attn.to_out.0", d, d)
    p += lin("attn.to_add_out", d, d)
    for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
        p.append((f"attn.{n}.weight", (hd,)))
    for s in ("img_mlp", "txt_mlp"):
        p += lin(f"{s}.net.0.proj", f, d)
        p += lin(f"{s}.net.2", d, f)
    return p


def embed_params(shape: QwenShape) -> list[tuple[str, tuple]]:
    d = shape.hidden
    lin = lambda n, o, i: [(f"{n}.weight", (o, i)), (f"{n}.bias", (o,))]  # noqa: E731
    p = []
    p += lin("img_in", d, shape.in_channels)
    p.append(("txt_norm.weight", (shape.txt_dim,)))
    p += lin("txt_in", d, shape.txt_dim)
    p += lin("time_text_embed.timestep_embedder.linear_1", d, 256)
    p += lin("time_text_embed.timestep_embedder.linear_2", d, d)
    p += lin("norm_out.linear", 2 * d, d)
    p += lin("proj_out", shape.out_channels, d)
    return p


def _is_norm_weight(name: str) -> bool:
    return name.endswith(".weight") and (".norm_" in name or name.startswith("txt_norm."))


def make_params(spec, seed: int, std: float = 0.02, dtype=torch.bfloat16) -> dict:
    """One parameter group: RMSNorm weights ones, the rest N(0, std) drawn in spec order from
    torch.Generator(seed), rounded to `dtype` and returned in fp32."""
    g = torch.Generator().manual_seed(int(seed))
    out = {}
    for name, shp in spec:
        t = torch.ones(shp) if _is_norm_weight(name) and len(shp) == 1 else _draw(g, shp, std)
        out[name] = t.to(dtype).float()
    return out


def block_weights(shape: QwenShape, seed: int, index: int, **kw) -> dict:
    return make_params(block_params(shape), seed + index, **kw)


def embed_weights(shape: QwenShape, seed: int, **kw) -> dict:
    return make_params(embed_params(shape), seed + EMBED_SEED_OFFSET, **kw)


# ------------------------------------------------------------------------------------ RoPE
def _axis_angles(index: torch.Tensor, dim: int, theta: int) -> torch.Tensor:
    """QwenEmbedRope.rope_params: outer(index, theta^-(2i/dim)) in fp32, [len(index), dim/2]."""
    inv = 1.0 / torch.pow(torch.tensor(float(theta)),
                          torch.arange(0, dim, 2, dtype=torch.float32).div(dim))
    return torch.outer(index.to(torch.float32), inv)


def _centred(n: int) -> torch.Tensor:
    """scale_rope positions of one image axis: -(n - n // 2) .. -1, then 0 .. n // 2 - 1."""
    return torch.cat([torch.arange(-(n - n // 2), 0), torch.arange(0, n // 2)])


def pos_embed(h: int, w: int, txt_len: int, axes=(16, 56, 56), theta=10000):
    """(cos, sin) fp32 [txt_len + h * w, sum(axes)] for the joint [txt | img] sequence, each
    angle repeated for its interleaved pair (modeling_qwen_image.py:46-49)."""
    a0, a1, a2 = axes
    hh, ww = torch.meshgrid(_centred(h), _centred(w), indexing="ij")
    img = torch.cat([_axis_angles(torch.zeros(h * w), a0, theta),
                     _axis_angles(hh.reshape(-1), a1, theta),
                     _axis_angles(ww.reshape(-1), a2, theta)], dim=1)
    start = max(h // 2, w // 2)
    p = torch.arange(start, start + txt_len)
    txt = torch.cat([_axis_angles(p, a0, theta), _axis_angles(p, a1, theta),
                     _axis_angles(p, a2, theta)], dim=1)
    ang = torch.cat([txt, img], dim=0)
    return (torch.cos(ang).repeat_interleave(2, dim=-1),
            torch.sin(ang).repeat_interleave(2, dim=-1))


# ------------------------------------------------------------------------------------ block
def _heads(x, shape: QwenShape):
    b, s, _ = x.shape
    return x.view(b, s, shape.heads, shape.head_dim).transpose(1, 2)


def _masked_joint_attention(q_img, k_img, v_img, q_txt, k_txt, v_txt, valid: int):
    """modeling_qwen_image.py:493-552 at cp = 1: keys and queries ordered [image | text], every
    query attends to the key prefix [0, S_img + valid) through the op's bounds (bound_min 0,
    bound_max S_img + valid), heads folded into the batch; the output is put back in
    [text | image] order. In [B, H, S, d]; out [B, H, S_txt + S_img, d]."""
    q = torch.cat([q_img, q_txt], dim=2)
    k = torch.cat([k_img, k_txt], dim=2)
    v = torch.cat([v_img, v_txt], dim=2)
    b, h, s_q, d = q.shape
    n_img = q_img.shape[2]
    bound_max = torch.full((b * h, s_q, 1), n_img + int(valid), dtype=torch.int32)
    out = ops.attention(q.reshape(b * h, s_q, d), k.reshape(b * h, -1, d),
                        v.reshape(b * h, -1, d), scale=1 / math.sqrt(d),
                        bound_min=torch.zeros_like(bound_max), bound_max=bound_max)
    out = out.reshape(b, h, s_q, d)
    return torch.cat([out[:, :, n_img:], out[:, :, :n_img]], dim=2)


def block(w: dict, hidden, context, temb, cos, sin, shape: QwenShape, quant=None,
          act_dtype=None, store=None, mods=None, text_valid_len=None):
    """One joint block; returns (context, hidden). `quant` = "mx" puts the MX targets through
    the MXFP8 law; `act_dtype` rounds their activations first (a bf16 device quantizes the bf16
    tensor). `store` (a dtype) rounds every activation the device keeps in memory to it;
    `mods` = (image [1, 6D], text [1, 6D]) replaces the computed modulation vectors.
    `text_valid_len` (an int) masks the text keys from that index on, the reference's masked
    joint attention for a right-padded prompt (modeling_qwen_image.py:493-552)."""
    L = ops.linear
    Q = qlinear(quant, act_dtype)
    R = ops.rounder(store)
    lin = lambda n, x: (Q if n in MX_TARGETS else L)(x, w[f"{n}.weight"], w[f"{n}.bias"])  # noqa: E731
    silu_t = torch.nn.functional.silu(temb)
    if mods is None:
        mods = (L(silu_t, w["img_mod.1.weight"], w["img_mod.1.bias"]),
                L(silu_t, w["txt_mod.1.weight"], w["txt_mod.1.bias"]))
    i_sh1, i_sc1, i_g1, i_sh2, i_sc2, i_g2 = R(mods[0]).chunk(6, dim=1)
    t_sh1, t_sc1, t_g1, t_sh2, t_sc2, t_g2 = R(mods[1]).chunk(6, dim=1)

    nx = R(ops.ada_modulate(hidden, i_sh1, i_sc1))
    nc = R(ops.ada_modulate(context, t_sh1, t_sc1))
    q, k, v = (_heads(R(lin(f"attn.{n}", nx)), shape) for n in ("to_q", "to_k", "to_v"))
    cq, ck, cv = (_heads(R(lin(f"attn.{n}", nc)), shape)
                  for n in ("add_q_proj", "add_k_proj", "add_v_proj"))
    q = ops.rms_norm_fp32(q, w["attn.norm_q.weight"], 1e-6)
    k = ops.rms_norm_fp32(k, w["attn.norm_k.weight"], 1e-6)
    cq = ops.rms_norm_fp32(cq, w["attn.norm_added_q.weight"], 1e-6)
    ck = ops.rms_norm_fp32(ck, w["attn.norm_added_k.weight"], 1e-6)
    st = context.shape[1]
    rope = lambda x, c, s: R(ops.apply_rotary_emb_fp32(x, c[None, None], s[None, None]))  # noqa: E731
    q_img, k_img = rope(q, cos[st:], sin[st:]), rope(k, cos[st:], sin[st:])
    q_txt, k_txt = rope(cq, cos[:st], sin[:st]), rope(ck, cos[:st], sin[:st])
    b, hh, _, d = q.shape
    if text_valid_len is None:
        qj, kj, vj = (torch.cat(p, dim=2) for p in ((q_txt, q_img), (k_txt, k_img), (cv, v)))
        s = qj.shape[2]
        o = ops.attention(qj.reshape(b * hh, s, d), kj.reshape(b * hh, s, d),
                          vj.reshape(b * hh, s, d), scale=1 / math.sqrt(d)).reshape(b, hh, s, d)
    else:
        o = _masked_joint_attention(q_img, k_img, v, q_txt, k_txt, cv, int(text_valid_len))
        s = o.shape[2]
    o = R(o.transpose(1, 2).reshape(b, s, hh * d))
    c_attn = lin("attn.to_add_out", o[:, :st])
    x_attn = lin("attn.to_out.0", o[:, st:])

    hidden = R(hidden + i_g1[:, None] * x_attn)
    context = R(context + t_g1[:, None] * c_attn)
    P = gelu_input_rounder(quant, store)  # the per-token fp8 law's GELU point
    nx2 = R(ops.ada_modulate(hidden, i_sh2, i_sc2))
    hidden = R(hidden + i_g2[:, None] * lin("img_mlp.net.2",
                                            R(ops.gelu_tanh(P(lin("img_mlp.net.0.proj", nx2))))))
    nc2 = R(ops.ada_modulate(context, t_sh2, t_sc2))
    context = R(context + t_g2[:, None] * lin("txt_mlp.net.2",
                                              R(ops.gelu_tanh(P(lin("txt_mlp.net.0.proj", nc2))))))
    return context, hidden


# ------------------------------------------------------------------------------------ model
def time_embed(ew: dict, timestep, model_dtype=torch.float32, store=None):
    """The timestep projection: the model casts t / 1000 to its dtype, the sinusoid scales it
    by 1000 (256 channels, cos first, shift 0), then linear_1 - SiLU - linear_2. `store`
    rounds the sinusoid and both linears' outputs as a device holding them in that dtype."""
    L = ops.linear
    R = ops.rounder(store)
    t = timestep.to(model_dtype).float() * 1000.0
    tp = R(ops.timestep_embedding(t, 256, flip_sin_to_cos=True, downscale_freq_shift=0))
    h = R(L(tp, ew["time_text_embed.timestep_embedder.linear_1.weight"],
            ew["time_text_embed.timestep_embedder.linear_1.bias"]))
    return R(L(torch.nn.functional.silu(h), ew["time_text_embed.timestep_embedder.linear_2.weight"],
               ew["time_text_embed.timestep_embedder.linear_2.bias"]))


def forward(shape: QwenShape, seed: int, latents, text, timestep, img_hw, weights=None,
            dtype=torch.bfloat16, model_dtype=torch.float32, quant=None, act_dtype=None,
            text_valid_len=None, store=None):
    """One denoise step: latents [B, h*w, in_ch] (packed 2x2 patches), text [B, S_txt,
    txt_dim] (the text encoder's hidden states), timestep t / 1000 [B] -> [B, h*w, out_ch].
    Blocks are drawn one at a time unless `weights` = (embed, [block...]) is given.
    `text_valid_len` masks a right-padded prompt's padding keys in every block (the
    reference's text_valid_len path, modeling_qwen_image.py:579-601,738-739). `store` rounds
    what a device keeps in that dtype, as in block()."""
    ew = weights[0] if weights else embed_weights(shape, seed, dtype=dtype)
    L = ops.linear
    R = ops.rounder(store)
    hidden = R(L(latents, ew["img_in.weight"], ew["img_in.bias"]))
    context = embed_text(ew, text, store)
    temb = time_embed(ew, timestep, model_dtype, store)
    cos, sin = pos_embed(img_hw[0], img_hw[1], text.shape[1], shape.axes, shape.theta)
    for i in range(shape.n_blocks):
        w = weights[1][i] if weights else block_weights(shape, seed, i, dtype=dtype)
        context, hidden = block(w, hidden, context, temb, cos, sin, shape, quant, act_dtype,
                                store=store, text_valid_len=text_valid_len)
    return final_layer(ew, hidden, temb, store)


def embed_text(ew: dict, text, store=None):
    """txt_norm (RMSNorm over the text encoder's width, eps 1e-6, the fp32 law) then txt_in:
    text [B, S_txt, txt_dim] -> [B, S_txt, D]. `store` rounds the normalised text and the
    result as a device holding them in that dtype."""
    R = ops.rounder(store)
    n = R(ops.rms_norm_fp32(text, ew["txt_norm.weight"], 1e-6))
    return R(ops.linear(n, ew["txt_in.weight"], ew["txt_in.bias"]))


def final_layer(ew: dict, hidden, temb, store=None):
    """AdaLayerNormContinuous norm_out (difflet/layers/normalization.py:150-190: emb =
    linear(SiLU(temb)), chunked scale first, then shift; LayerNorm without affine, eps 1e-6)
    and proj_out: hidden [B, S_img, D], temb [B, D] -> [B, S_img, out_ch]."""
    L = ops.linear
    R = ops.rounder(store)
    emb = R(L(torch.nn.functional.silu(temb), ew["norm_out.linear.weight"], ew["norm_out.linear.bias"]))
    scale, shift = emb.chunk(2, dim=1)  # AdaLayerNormContinuous: scale first
    hidden = R(ops.layer_norm(hidden) * (1 + scale)[:, None] + shift[:, None])
    return L(hidden, ew["proj_out.weight"], ew["proj_out.bias"])


def synthetic_inputs(shape: QwenShape, seed: int, img_hw, txt_len, batch: int = 1):
    """latents [B, h*w, in_ch] and text [B, txt_len, txt_dim] ~ N(0, 1); timestep t / 1000 with
    t ~ U[0, 1000)."""
    g = torch.Generator().manual_seed(int(seed))
    h, w = img_hw
    latents = torch.randn(batch, h * w, shape.in_channels, generator=g)
    text = torch.randn(batch, txt_len, shape.txt_dim, generator=g)
    t = torch.rand(batch, generator=g) * 1000.0
    return {"latents": latents, "text": text, "timestep": t / 1000.0}
