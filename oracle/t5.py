"""The T5 text encoders restated in fp32 on the CPU: FLUX's T5-XXL (text_encoder_2) and Wan's
UMT5-XXL, with seeded random weights. Test infrastructure only (see oracle/__init__.py).

Follows, at tp = 1 and in eval mode (dropout off):
  T5LayerNorm                :difflet/models/flux/t5/modeling_t5.py:61-83 (RMSNorm without
                              mean centring, fp32 variance, weight last)
  _relative_position_bucket  :modeling_t5.py:200-248, difflet/models/wan/umt5/
                              modeling_umt5.py:196-223 (bidirectional: half the buckets for
                              keys after the query, half exact and half logarithmic up to
                              max_distance)
  compute_bias               :modeling_t5.py:250-269, modeling_umt5.py:225-242
                              (table[bucket(k - q)] as [1, heads, q, k])
  attention                  :modeling_t5.py:271-414, modeling_umt5.py:244-281 (no 1/sqrt(d)
                              scale; scores + position bias (+ padding mask); fp32 softmax;
                              o projection)
  gated FFN                  :modeling_t5.py:114-150, modeling_umt5.py:101-130
                              (gelu_new(wi_0 h) * wi_1 h, then wo)
  pre-norm residual layers   :modeling_t5.py:153-168,417-448; modeling_umt5.py:133-145,284-305
  stack                      :modeling_t5.py:542-722 (block 0 owns the bias table and every
                              block reuses its bias; the encoder model asserts no mask),
                              modeling_umt5.py:336-369 (every block owns a table; the (B, S)
                              padding mask becomes (1 - mask) * finfo.min on the keys)

`store` (a dtype or None) rounds the activations where a device that keeps them in that dtype
stores them (ops.rounder), so a bf16 device run is compared against the same rounding points.

Weights: N(0, std) per parameter from torch.Generator(seed + index) in param_shapes order, the
stds of transformers' T5 initialisation (q (d_model d_kv)^-1/2, k / v / wi d_model^-1/2, o
(heads d_kv)^-1/2, wo d_ff^-1/2, bias tables d_model^-1/2, embedding 1); norm weights
1 + N(0, 0.1) so that a dropped weight shows.
"""

from __future__ import annotations

import dataclasses
import math

import torch

from oracle import ops


@dataclasses.dataclass(frozen=True)
class T5Shape:
    vocab: int = 32128
    d_model: int = 4096
    d_kv: int = 64
    d_ff: int = 10240
    heads: int = 64
    layers: int = 24
    buckets: int = 32
    max_distance: int = 128
    eps: float = 1e-6
    per_layer_bias: bool = False  # UMT5: every block owns its relative bias table

    @property
    def inner(self) -> int:
        return self.heads * self.d_kv


T5_XXL = T5Shape()                                          # google/t5-v1_1-xxl (FLUX.1)
UMT5_XXL = T5Shape(vocab=256384, per_layer_bias=True)       # umt5-xxl (Wan 2.x)


def param_shapes(shape: T5Shape) -> list[tuple[str, tuple]]:
    """Hugging Face T5 / UMT5 encoder keys, the layout the reference loads key for key."""
    d, inner, f = shape.d_model, shape.inner, shape.d_ff
    p = [("shared.weight", (shape.vocab, d))]
    for i in range(shape.layers):
        a = f"encoder.block.{i}.layer.0."
        p += [(a + "SelfAttention.q.weight", (inner, d)), (a + "SelfAttention.k.weight", (inner, d)),
              (a + "SelfAttention.v.weight", (inner, d)), (a + "SelfAttention.o.weight", (d, inner))]
        if i == 0 or shape.per_layer_bias:
            p.append((a + "SelfAttention.relative_attention_bias.weight", (shape.buckets, shape.heads)))
        p.append((a + "layer_norm.weight", (d,)))
        m = f"encoder.block.{i}.layer.1."
        p += [(m + "DenseReluDense.wi_0.weight", (f, d)), (m + "DenseReluDense.wi_1.weight", (f, d)),
              (m + "DenseReluDense.wo.weight", (d, f)), (m + "layer_norm.weight", (d,))]
    p.append(("encoder.final_layer_norm.weight", (d,)))
    return p


def _std(name: str, shape: T5Shape) -> float:
    if name == "shared.weight":
        return 1.0
    if name.endswith("q.weight"):
        return (shape.d_model * shape.d_kv) ** -0.5
    if name.endswith("o.weight") and "SelfAttention" in name:
        return shape.inner ** -0.5
    if name.endswith("wo.weight"):
        return shape.d_ff ** -0.5
    return shape.d_model ** -0.5


def weights(shape: T5Shape, seed: int, dtype: torch.dtype | None = None) -> dict[str, torch.Tensor]:
    """fp32 parameters (values rounded through `dtype` when given)."""
    r = ops.rounder(dtype)
    out = {}
    for idx, (name, shp) in enumerate(param_shapes(shape)):
        g = torch.Generator().manual_seed(seed * 1009 + idx)
        x = torch.randn(shp, generator=g, dtype=torch.float32)
        x = 1.0 + 0.1 * x if name.endswith("layer_norm.weight") else x * _std(name, shape)
        out[name] = r(x)
    return out


def relative_position_bucket(rel: torch.Tensor, num_buckets: int, max_distance: int) -> torch.Tensor:
    """modeling_t5.py:200-248 (bidirectional=True, the encoder's): keys after the query use the
    upper half of the buckets; within a half, distances below a quarter of the buckets are exact
    and the rest are binned logarithmically up to max_distance (the last bin takes the rest)."""
    half = num_buckets // 2
    base = (rel > 0).to(torch.long) * half
    dist = rel.abs()
    exact = half // 2
    logb = exact + (torch.log(dist.float() / exact) / math.log(max_distance / exact)
                    * (half - exact)).to(torch.long)
    logb = torch.clamp(logb, max=half - 1)
    return base + torch.where(dist < exact, dist, logb)


def position_bias(table: torch.Tensor, seq_q: int, seq_k: int, shape: T5Shape) -> torch.Tensor:
    """compute_bias (modeling_t5.py:250-269): [1, heads, seq_q, seq_k]."""
    rel = torch.arange(seq_k)[None, :] - torch.arange(seq_q)[:, None]
    b = relative_position_bucket(rel, shape.buckets, shape.max_distance)
    return table[b].permute(2, 0, 1).unsqueeze(0)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """T5LayerNorm in fp32 (modeling_t5.py:70-83)."""
    var = x.pow(2).mean(-1, keepdim=True)
    return w * (x * torch.rsqrt(var + eps))


def gelu_new(x: torch.Tensor) -> torch.Tensor:
    """transformers' gelu_new (the config's dense_act_fn): the tanh approximation."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x.pow(3))))


def padding_mask(attention_mask: torch.Tensor) -> torch.Tensor:
    """modeling_umt5.py:354-358 in fp32: (B, S) {0, 1} -> additive (B, 1, 1, S)."""
    m = attention_mask[:, None, None, :].to(torch.float32)
    return (1.0 - m) * torch.finfo(torch.float32).min


def encode(w: dict[str, torch.Tensor], shape: T5Shape, input_ids: torch.Tensor,
           attention_mask: torch.Tensor | None = None, store=None) -> torch.Tensor:
    """last_hidden_state [B, S, d_model] of the encoder stack."""
    if attention_mask is not None and not shape.per_layer_bias:
        raise ValueError("the T5 encoder model takes no attention mask (modeling_t5.py:787)")
    r = ops.rounder(store)
    b, s = input_ids.shape
    x = w["shared.weight"][input_ids]
    add = padding_mask(attention_mask) if attention_mask is not None else None
    bias = None
    for i in range(shape.layers):
        p = f"encoder.block.{i}.layer."
        if bias is None or shape.per_layer_bias:
            bias = position_bias(w[p + "0.SelfAttention.relative_attention_bias.weight"], s, s, shape)
            if add is not None:
                bias = bias + add
        n = r(rms_norm(x, w[p + "0.layer_norm.weight"], shape.eps))
        heads = lambda t: t.view(b, s, shape.heads, shape.d_kv).transpose(1, 2)  # noqa: E731
        q, k, v = (heads(r(n @ w[p + f"0.SelfAttention.{c}.weight"].T)) for c in "qkv")
        scores = q @ k.transpose(-1, -2) + bias
        probs = torch.softmax(scores, dim=-1)
        a = r((probs @ v).transpose(1, 2).reshape(b, s, shape.inner))
        x = r(x + a @ w[p + "0.SelfAttention.o.weight"].T)
        n = r(rms_norm(x, w[p + "1.layer_norm.weight"], shape.eps))
        g = r(gelu_new(r(n @ w[p + "1.DenseReluDense.wi_0.weight"].T))
              * r(n @ w[p + "1.DenseReluDense.wi_1.weight"].T))
        x = r(x + g @ w[p + "1.DenseReluDense.wo.weight"].T)
    return r(rms_norm(x, w["encoder.final_layer_norm.weight"], shape.eps))
