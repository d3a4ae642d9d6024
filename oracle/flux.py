"""FLUX.1 transformer restated from the reference modeling code, fp32 on the CPU, with seeded
random weights. Test infrastructure only (see oracle/__init__.py).

Follows difflet/models/flux/modeling_flux.py at tp = 1 on the `cpu` backend (no context /
sequence / CFG parallelism; `hardware` is CPU, so attention goes through
`attention_wrapper_sharded_without_swap`, :119-153):
  model forward       :364-613   (x_embedder, timestep*1000, guidance*1000, time_text_embed,
                                  context_embedder, 19 double blocks, concat [txt | img],
                                  38 single blocks, image slice, norm_out, proj_out)
  double block        :796-867
  single block        :696-736   (proj_out as the attn/mlp column halves, summed, + bias)
  attention           :1190-1462 (q/k/v, per-head RMSNorm, text-first concat, RoPE, SDPA)
  FFN                 :870-949   (GELU-tanh MLP)
  adaLN-Zero(-Single) difflet/layers/normalization.py:38-147, AdaLN-Continuous :150-190
  time/text embedding difflet/layers/embeddings.py:247-398,422-473

Weights are parameters named as diffusers' FluxTransformer2DModel names them, drawn
N(0, std) per block from torch.Generator(seed + block index) in a fixed order, then rounded to
the model dtype (the device model holds them in that dtype; the oracle computes in fp32 on the
rounded values). RMSNorm weights are ones.
"""

from __future__ import annotations

import dataclasses
import math

import torch

from oracle import ops


@dataclasses.dataclass(frozen=True)
class FluxShape:
    hidden: int = 3072
    heads: int = 24
    head_dim: int = 128
    mlp_ratio: int = 4
    n_double: int = 19
    n_single: int = 38
    in_channels: int = 64
    out_channels: int = 64
    txt_dim: int = 4096
    pooled_dim: int = 768
    axes: tuple = (16, 56, 56)
    guidance: bool = True

    @property
    def mlp(self) -> int:
        return self.hidden * self.mlp_ratio


FLUX_DEV = FluxShape()
EMBED_SEED_OFFSET = 100_000  # embedders / final layers draw from seed + this


def _draw(g, shape, std):
    return torch.randn(shape, generator=g, dtype=torch.float32) * std


def double_block_params(shape: FluxShape) -> list[tuple[str, tuple]]:
    d, f, hd = shape.hidden, shape.mlp, shape.head_dim
    lin = lambda n, o, i: [(f"{n}.weight", (o, i)), (f"{n}.bias", (o,))]  # noqa: E731
    p = []
    p += lin("norm1.linear", 6 * d, d)
    p += lin("norm1_context.linear", 6 * d, d)
    for n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj"):
        p += lin(f"attn.{n}", d, d)
    p += lin("attn.to_out.0", d, d)
    p += lin("attn.to_add_out", d, d)
    for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
        p.append((f"attn.{n}.weight", (hd,)))
    p += lin("ff.net.0.proj", f, d)
    p += lin("ff.net.2", d, f)
    p += lin("ff_context.net.0.proj", f, d)
    p += lin("ff_context.net.2", d, f)
    return p


def single_block_params(shape: FluxShape) -> list[tuple[str, tuple]]:
    d, f, hd = shape.hidden, shape.mlp, shape.head_dim
    lin = lambda n, o, i: [(f"{n}.weight", (o, i)), (f"{n}.bias", (o,))]  # noqa: E731
    p = []
    p += lin("norm.linear", 3 * d, d)
    p += lin("proj_mlp", f, d)
    for n in ("to_q", "to_k", "to_v"):
        p += lin(f"attn.{n}", d, d)
    for n in ("norm_q", "norm_k"):
        p.append((f"attn.{n}.weight", (hd,)))
    p += lin("proj_out", d, d + f)  # diffusers' fused [attn | mlp] weight
    return p


def embed_params(shape: FluxShape) -> list[tuple[str, tuple]]:
    d = shape.hidden
    lin = lambda n, o, i: [(f"{n}.weight", (o, i)), (f"{n}.bias", (o,))]  # noqa: E731
    p = []
    p += lin("x_embedder", d, shape.in_channels)
    p += lin("context_embedder", d, shape.txt_dim)
    p += lin("time_text_embed.timestep_embedder.linear_1", d, 256)
    p += lin("time_text_embed.timestep_embedder.linear_2", d, d)
    if shape.guidance:
        p += lin("time_text_embed.guidance_embedder.linear_1", d, 256)
        p += lin("time_text_embed.guidance_embedder.linear_2", d, d)
    p += lin("time_text_embed.text_embedder.linear_1", d, shape.pooled_dim)
    p += lin("time_text_embed.text_embedder.linear_2", d, d)
    p += lin("norm_out.linear", 2 * d, d)
    p += lin("proj_out", shape.out_channels, d)
    return p


def make_params(spec, seed: int, std: float = 0.02, dtype=torch.bfloat16) -> dict:
    """Draws one parameter group: RMSNorm weights are ones, everything else N(0, std), rounded
    to `dtype` (the model dtype) and returned in fp32."""
    g = torch.Generator().manual_seed(int(seed))
    out = {}
    for name, shp in spec:
        if ".norm_" in name and name.endswith(".weight") and len(shp) == 1:
            t = torch.ones(shp)
        else:
            t = _draw(g, shp, std)
        out[name] = t.to(dtype).float()
    return out


def double_block_weights(shape: FluxShape, seed: int, index: int, **kw) -> dict:
    return make_params(double_block_params(shape), seed + index, **kw)


def single_block_weights(shape: FluxShape, seed: int, index: int, **kw) -> dict:
    return make_params(single_block_params(shape), seed + shape.n_double + index, **kw)


def embed_weights(shape: FluxShape, seed: int, **kw) -> dict:
    return make_params(embed_params(shape), seed + EMBED_SEED_OFFSET, **kw)


# ------------------------------------------------------------------------------------ blocks
def qlinear(quant, act_dtype=None):
    """The block linear of a given format: fp32 F.linear, or the fp8 laws applied to both
    operands (codes as the device produces them) with the product in fp32. `act_dtype`
    rounds the activation to that dtype first, as a device that keeps bf16 activations
    quantizes the bf16 tensor."""
    if quant is None:
        return ops.linear
    if quant not in ("fp8", "mx"):
        raise ValueError(quant)
    from oracle import fp8 as ofp8
    from oracle import mx as omx

    def lin(x, w, b=None):
        if act_dtype is not None:
            x = x.to(act_dtype).float()
        # the torch twins of the numpy laws (pinned bit-exact against them), threaded
        if quant == "fp8":
            return ofp8.fp8_linear_torch(x, w, b)
        y = omx.fake_quantize_mx_torch(x) @ omx.fake_quantize_mx_torch(w).T
        return y if b is None else y + b

    return lin


def gelu_input_rounder(quant, store):
    """Where the MLP's GELU reads its input. Under the per-token fp8 law the producing GEMM
    stores the pre-activation (rounded to `store`) and the next GEMM's activation quantizer
    applies the GELU (difflet_rocm_quantize_fp8_rowwise_gelu); otherwise the GELU takes the
    fp32 GEMM output (a GELU epilogue)."""
    return ops.rounder(store) if quant == "fp8" else (lambda x: x)


def _heads(x, shape: FluxShape):
    b, s, _ = x.shape
    return x.view(b, s, shape.heads, shape.head_dim).transpose(1, 2)


def _rope(x, cos, sin):
    return ops.apply_rotary_emb_fp32(x, cos[None, None], sin[None, None])


def double_block(w: dict, hidden, context, temb, cos, sin, shape: FluxShape,
                 rms_law=ops.rms_norm_cpu_law, quant=None, act_dtype=None, store=None,
                 mods=None):
    """modeling_flux.py:796-867 with NeuronFluxAttention (:1190-1462). Returns (context, hidden).
    `quant` ("fp8" / "mx") quantizes every block linear but the adaLN ones. `store` (a dtype)
    rounds every activation the device keeps in memory to it (modulation vectors, LayerNorm
    outputs, projections before and after q/k norm + RoPE, attention output, MLP hidden, the
    residual stream); `mods` = (image [1, 6D], context [1, 6D]) replaces the computed
    modulation vectors."""
    L = ops.linear
    Q = qlinear(quant, act_dtype)
    R = ops.rounder(store)
    silu_t = torch.nn.functional.silu(temb)
    if mods is None:
        mods = (L(silu_t, w["norm1.linear.weight"], w["norm1.linear.bias"]),
                L(silu_t, w["norm1_context.linear.weight"], w["norm1_context.linear.bias"]))
    emb, cemb = R(mods[0]), R(mods[1])
    sh_msa, sc_msa, g_msa, sh_mlp, sc_mlp, g_mlp = emb.chunk(6, dim=1)
    c_sh_msa, c_sc_msa, c_g_msa, c_sh_mlp, c_sc_mlp, c_g_mlp = cemb.chunk(6, dim=1)
    nx = R(ops.ada_modulate(hidden, sh_msa, sc_msa))
    nc = R(ops.ada_modulate(context, c_sh_msa, c_sc_msa))

    a = lambda n, x: R(Q(x, w[f"attn.{n}.weight"], w[f"attn.{n}.bias"]))  # noqa: E731
    q, k, v = _heads(a("to_q", nx), shape), _heads(a("to_k", nx), shape), _heads(a("to_v", nx), shape)
    q = rms_law(q, w["attn.norm_q.weight"], 1e-6)
    k = rms_law(k, w["attn.norm_k.weight"], 1e-6)
    cq, ck, cv = (_heads(a("add_q_proj", nc), shape), _heads(a("add_k_proj", nc), shape),
                  _heads(a("add_v_proj", nc), shape))
    cq = rms_law(cq, w["attn.norm_added_q.weight"], 1e-6)
    ck = rms_law(ck, w["attn.norm_added_k.weight"], 1e-6)
    q = torch.cat([cq, q], dim=2)
    k = torch.cat([ck, k], dim=2)
    v = torch.cat([cv, v], dim=2)
    q, k = R(_rope(q, cos, sin)), R(_rope(k, cos, sin))
    o = R(_attend(q, k, v, shape))
    st = context.shape[1]
    c_attn, x_attn = o[:, :st], o[:, st:]
    x_attn = Q(x_attn, w["attn.to_out.0.weight"], w["attn.to_out.0.bias"])
    c_attn = Q(c_attn, w["attn.to_add_out.weight"], w["attn.to_add_out.bias"])

    hidden = R(hidden + g_msa[:, None] * x_attn)
    nx2 = R(ops.ada_modulate(hidden, sh_mlp, sc_mlp))
    P = gelu_input_rounder(quant, store)
    ff = Q(R(ops.gelu_tanh(P(Q(nx2, w["ff.net.0.proj.weight"], w["ff.net.0.proj.bias"])))),
           w["ff.net.2.weight"], w["ff.net.2.bias"])
    hidden = R(hidden + g_mlp[:, None] * ff)

    context = R(context + c_g_msa[:, None] * c_attn)
    nc2 = R(ops.ada_modulate(context, c_sh_mlp, c_sc_mlp))
    cff = Q(R(ops.gelu_tanh(P(Q(nc2, w["ff_context.net.0.proj.weight"],
                                w["ff_context.net.0.proj.bias"])))),
            w["ff_context.net.2.weight"], w["ff_context.net.2.bias"])
    context = R(context + c_g_mlp[:, None] * cff)
    return context, hidden


def _attend(q, k, v, shape: FluxShape):
    """attention_wrapper_sharded_without_swap (modeling_flux.py:119-153): heads folded into the
    batch, scale 1/sqrt(d), output back to [B, S, H*d]."""
    b, h, s, d = q.shape
    o = ops.attention(q.reshape(b * h, s, d), k.reshape(b * h, -1, d), v.reshape(b * h, -1, d),
                      scale=1 / math.sqrt(d))
    return o.reshape(b, h, s, d).transpose(1, 2).reshape(b, s, h * d)


def single_block(w: dict, hidden, temb, cos, sin, shape: FluxShape, rms_law=ops.rms_norm_cpu_law,
                 quant=None, act_dtype=None, store=None, mods=None):
    """modeling_flux.py:696-736: proj_out over [attn | mlp] as two column halves + bias. Under
    `quant` the proj_out is quantized as the one [D, D + mlp] linear the device runs (the fp8
    per-channel scale spans both halves; for MXFP8 it equals quantizing the halves separately,
    the attention half's K being a whole number of 512-wide swizzle tiles). `store` and `mods`
    ([1, 3D]) as in double_block."""
    L = ops.linear
    Q = qlinear(quant, act_dtype)
    R = ops.rounder(store)
    d = shape.hidden
    if mods is None:
        mods = L(torch.nn.functional.silu(temb), w["norm.linear.weight"], w["norm.linear.bias"])
    shift, scale, gate = R(mods).chunk(3, dim=1)
    nh = R(ops.ada_modulate(hidden, shift, scale))
    mlp = R(ops.gelu_tanh(gelu_input_rounder(quant, store)(
        Q(nh, w["proj_mlp.weight"], w["proj_mlp.bias"]))))
    a = lambda n: R(Q(nh, w[f"attn.{n}.weight"], w[f"attn.{n}.bias"]))  # noqa: E731
    q, k, v = _heads(a("to_q"), shape), _heads(a("to_k"), shape), _heads(a("to_v"), shape)
    q = rms_law(q, w["attn.norm_q.weight"], 1e-6)
    k = rms_law(k, w["attn.norm_k.weight"], 1e-6)
    q, k = R(_rope(q, cos, sin)), R(_rope(k, cos, sin))
    o = R(_attend(q, k, v, shape))
    wp = w["proj_out.weight"]
    if quant is None:
        out = L(o, wp[:, :d]) + L(mlp, wp[:, d:])
    else:
        out = Q(torch.cat([o, mlp], dim=-1), wp)
    return R(hidden + gate[:, None] * (out + w["proj_out.bias"]))


# ------------------------------------------------------------------------------------ model
def time_text_embed(ew: dict, timestep, guidance, pooled, shape: FluxShape):
    """NeuronCombinedTimestepGuidanceTextProjEmbeddings (difflet/layers/embeddings.py:247-281);
    timestep / guidance are already multiplied by 1000 (modeling_flux.py:477-479)."""
    L = ops.linear
    silu = torch.nn.functional.silu

    def mlp(prefix, x):
        h = L(x, ew[f"{prefix}.linear_1.weight"], ew[f"{prefix}.linear_1.bias"])
        return L(silu(h), ew[f"{prefix}.linear_2.weight"], ew[f"{prefix}.linear_2.bias"])

    tp = ops.timestep_embedding(timestep, 256, flip_sin_to_cos=True, downscale_freq_shift=0)
    emb = mlp("time_text_embed.timestep_embedder", tp)
    if shape.guidance:
        gp = ops.timestep_embedding(guidance, 256, flip_sin_to_cos=True, downscale_freq_shift=0)
        emb = emb + mlp("time_text_embed.guidance_embedder", gp)
    return emb + mlp("time_text_embed.text_embedder", pooled)


def forward(shape: FluxShape, seed: int, latents, text, pooled, timestep, guidance, img_hw,
            weights=None, rms_law=ops.rms_norm_cpu_law, dtype=torch.bfloat16,
            model_dtype=torch.float32, quant=None, rope_dtype=None):
    """One denoise step (modeling_flux.py:364-613). Block weights are drawn block by block
    (never all held) unless `weights` = (embed, double, single) is given, double / single
    being lists of block weights or callables returning block i's (fetched one at a time).
    `dtype` is the weights' storage dtype; `model_dtype` the model's torch dtype, which the
    reference casts timestep and guidance to and scales by 1000 in (:453-456,477-479); the
    compute itself is fp32. `rope_dtype` rounds the RoPE table to that dtype, as the
    reference's GPU adapter does when it stacks the table and casts it to the model dtype
    (difflet/backends/cuda/flux/transformer.py:184-188)."""
    ew = weights[0] if weights else embed_weights(shape, seed, dtype=dtype)
    L = ops.linear
    hidden = L(latents, ew["x_embedder.weight"], ew["x_embedder.bias"])
    t1000 = (timestep.to(model_dtype) * 1000).float()
    g1000 = (guidance.to(model_dtype) * 1000).float()
    temb = time_text_embed(ew, t1000, g1000, pooled, shape)
    context = L(text, ew["context_embedder.weight"], ew["context_embedder.bias"])
    ids = ops.flux_ids(text.shape[1], *img_hw)
    cos, sin = ops.flux_pos_embed(ids, shape.axes)
    if rope_dtype is not None:
        cos, sin = cos.to(rope_dtype).float(), sin.to(rope_dtype).float()
    for i in range(shape.n_double):
        w = _block(weights, 1, i) if weights else double_block_weights(shape, seed, i, dtype=dtype)
        context, hidden = double_block(w, hidden, context, temb, cos, sin, shape, rms_law, quant)
    hidden = torch.cat([context, hidden], dim=1)
    for i in range(shape.n_single):
        w = _block(weights, 2, i) if weights else single_block_weights(shape, seed, i, dtype=dtype)
        hidden = single_block(w, hidden, temb, cos, sin, shape, rms_law, quant)
    hidden = hidden[:, text.shape[1]:]
    emb = L(torch.nn.functional.silu(temb), ew["norm_out.linear.weight"], ew["norm_out.linear.bias"])
    scale, shift = emb.chunk(2, dim=1)  # AdaLN-Continuous: scale first (normalization.py:188)
    hidden = ops.layer_norm(hidden) * (1 + scale)[:, None] + shift[:, None]
    return L(hidden, ew["proj_out.weight"], ew["proj_out.bias"])


def _block(weights, part: int, i: int) -> dict:
    src = weights[part]
    return src(i) if callable(src) else src[i]


def synthetic_inputs(shape: FluxShape, seed: int, img_hw, txt_len, batch: int = 1):
    """Config inputs: latents [B, h*w, in_ch], text [B, txt_len, txt_dim], pooled
    [B, pooled_dim] ~ N(0, 1); timestep t/1000 with t ~ U[0, 1000); guidance 3.5."""
    g = torch.Generator().manual_seed(int(seed))
    h, w = img_hw
    latents = torch.randn(batch, h * w, shape.in_channels, generator=g)
    text = torch.randn(batch, txt_len, shape.txt_dim, generator=g)
    pooled = torch.randn(batch, shape.pooled_dim, generator=g)
    t = torch.rand(batch, generator=g) * 1000.0
    return {"latents": latents, "text": text, "pooled": pooled, "timestep": t / 1000.0,
            "guidance": torch.full((batch,), 3.5)}
