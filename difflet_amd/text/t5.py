"""The T5 text encoders on the gfx950 kernels: FLUX's T5-XXL (NeuronT5EncoderModel,
difflet/models/flux/t5/modeling_t5.py:725-799) and Wan's UMT5-XXL (WanUmT5EncoderModel,
difflet/models/wan/umt5/modeling_umt5.py:372-400), in bf16 or fp32 (the reference runs either:
difflet/backends/neuron/flux/text_encoder.py:10-16, difflet/backends/neuron/wan/
text_encoder.py:9-17).

Per block, 8 launches: RMSNorm -> [q|k|v] GEMM -> attention (head_dim 64, no score scale, the
relative position bias as an additive fp32 mask, q / k / v read in place from the projection
buffer) -> o projection + residual (GEMM epilogue) -> RMSNorm -> [wi_0|wi_1] GEMM -> gated GELU
-> wo + residual (GEMM epilogue). The bias [B or 1, heads, S, S] is built on the device from a
host-computed bucket per relative position: once per forward for T5 (block 0's table serves
every block, modeling_t5.py:550-555,682-685), per block for UMT5 (modeling_umt5.py:308-366),
with UMT5's key padding folded in as the lowest float (its (1 - mask) * finfo.min,
modeling_umt5.py:354-358; a row of padding only stays finite, as in the reference).

bf16 runs the bf16 GEMM and the MFMA attention kernel; fp32 the fp32 matrix-core GEMM and the
fp32 attention kernel. HBM layout (tokens B * S, D = d_model): x [BS, D] residual stream,
qkv [BS, 3 * heads * d_kv], att [BS, heads * d_kv], ff [BS, 2 d_ff], g [BS, d_ff].
"""

from __future__ import annotations

import dataclasses
import math
from typing import Callable

import torch

from difflet_amd import _lib, kernels


@dataclasses.dataclass(frozen=True)
class T5Config:
    """Encoder hyperparameters, Hugging Face config names (T5Config / UMT5Config)."""

    vocab_size: int = 32128
    d_model: int = 4096
    d_kv: int = 64
    d_ff: int = 10240
    num_heads: int = 64
    num_layers: int = 24
    relative_attention_num_buckets: int = 32
    relative_attention_max_distance: int = 128
    layer_norm_epsilon: float = 1e-6
    per_layer_bias: bool = False  # UMT5: every block owns a relative bias table

    @property
    def inner_dim(self) -> int:
        return self.num_heads * self.d_kv

    @classmethod
    def from_hf_dict(cls, raw: dict, *, umt5: bool) -> "T5Config":
        """From a config.json (the reference reads T5Config / WanUmT5Config the same way:
        modeling_umt5.py:90-94). Only the gated-GELU feed-forward is supported, as in the
        reference's UMT5 (modeling_umt5.py:79-84) and the T5 v1.1 checkpoints FLUX uses."""
        proj = raw.get("feed_forward_proj", "gated-gelu")
        if proj != "gated-gelu" or raw.get("dense_act_fn", "gelu_new") not in ("gelu_new", "gelu_pytorch_tanh"):
            raise NotImplementedError(f"only the gated tanh-GELU feed-forward is supported, got {proj}")
        names = {f.name for f in dataclasses.fields(cls)}
        return cls(**{k: v for k, v in raw.items() if k in names}, per_layer_bias=umt5)


T5_XXL = T5Config()                                          # google/t5-v1_1-xxl (FLUX.1)
UMT5_XXL = T5Config(vocab_size=256384, per_layer_bias=True)  # umt5-xxl (Wan 2.x)


def param_shapes(cfg: T5Config) -> dict[str, tuple]:
    """Hugging Face encoder keys (the reference loads them key for key)."""
    d, inner, f = cfg.d_model, cfg.inner_dim, cfg.d_ff
    p = {"shared.weight": (cfg.vocab_size, d)}
    for i in range(cfg.num_layers):
        a = f"encoder.block.{i}.layer.0."
        for c in "qkv":
            p[a + f"SelfAttention.{c}.weight"] = (inner, d)
        p[a + "SelfAttention.o.weight"] = (d, inner)
        if i == 0 or cfg.per_layer_bias:
            p[a + "SelfAttention.relative_attention_bias.weight"] = (
                cfg.relative_attention_num_buckets, cfg.num_heads)
        p[a + "layer_norm.weight"] = (d,)
        m = f"encoder.block.{i}.layer.1."
        p[m + "DenseReluDense.wi_0.weight"] = (f, d)
        p[m + "DenseReluDense.wi_1.weight"] = (f, d)
        p[m + "DenseReluDense.wo.weight"] = (d, f)
        p[m + "layer_norm.weight"] = (d,)
    p["encoder.final_layer_norm.weight"] = (d,)
    return p


def random_param_source(cfg: T5Config, seed: int, device, dtype=torch.bfloat16):
    """Parameters drawn on the device on demand with transformers' T5 initialisation stds
    (embedding 1, q (d_model d_kv)^-1/2, o (heads d_kv)^-1/2, wo d_ff^-1/2, the rest
    d_model^-1/2); norm weights 1 + N(0, 0.1). One generator per parameter, seeded from
    (seed, name)."""
    import zlib

    shapes = param_shapes(cfg)

    def std(name):
        if name == "shared.weight":
            return 1.0
        if name.endswith("q.weight"):
            return (cfg.d_model * cfg.d_kv) ** -0.5
        if name.endswith("SelfAttention.o.weight"):
            return cfg.inner_dim ** -0.5
        if name.endswith("wo.weight"):
            return cfg.d_ff ** -0.5
        return cfg.d_model ** -0.5

    def get(name: str) -> torch.Tensor:
        g = torch.Generator(device=device).manual_seed(seed * 1_000_003 + zlib.crc32(name.encode()))
        x = torch.randn(shapes[name], generator=g, device=device, dtype=torch.float32)
        x = 1.0 + 0.1 * x if name.endswith("layer_norm.weight") else x * std(name)
        return x.to(dtype)

    return get


def relative_position_buckets(seq_q: int, seq_k: int, num_buckets: int,
                              max_distance: int) -> torch.Tensor:
    """int32 [seq_q + seq_k - 1]: entry j is the bucket of relative position j - (seq_q - 1)
    (key minus query), by _relative_position_bucket with bidirectional=True
    (modeling_t5.py:200-248): keys after the query take the upper half of the buckets; within a
    half, distances below a quarter of the buckets are exact and longer ones are binned
    logarithmically up to max_distance. Computed on the host with the reference's own fp32 torch
    operations (the log and its truncation decide the bin edges), once per sequence length."""
    rel = torch.arange(-(seq_q - 1), seq_k, dtype=torch.long)
    half = num_buckets // 2
    upper = (rel > 0).to(torch.long) * half
    dist = rel.abs()
    exact = half // 2
    binned = exact + (torch.log(dist.float() / exact) / math.log(max_distance / exact)
                      * (half - exact)).to(torch.long)
    binned = torch.minimum(binned, torch.full_like(binned, half - 1))
    return (upper + torch.where(dist < exact, dist, binned)).to(torch.int32)


class T5Encoder:
    """The encoder stack on one device. param_source(name) -> tensor for the keys of
    param_shapes; forward(input_ids [B, S] int64, attention_mask [B, S] {0, 1} or None) ->
    last_hidden_state [B, S, d_model] in the model dtype."""

    def __init__(self, cfg: T5Config, param_source: Callable[[str], torch.Tensor], *,
                 dtype: torch.dtype = torch.bfloat16, device="cuda"):
        if dtype not in (torch.bfloat16, torch.float32):
            raise NotImplementedError(f"T5Encoder runs bf16 or fp32, not {dtype}")
        if cfg.d_kv not in (64, 128):
            raise NotImplementedError(f"attention head_dim {cfg.d_kv} (64 or 128 supported)")
        self.cfg, self.dtype = cfg, dtype
        self.device = torch.device(device)
        kt = 64 if dtype == torch.bfloat16 else 4  # the GEMMs' K multiple
        for k in (cfg.d_model, cfg.inner_dim, cfg.d_ff):
            if k % kt:
                raise NotImplementedError(f"width {k} is not a multiple of {kt}")

        def get(name):
            return param_source(name).to(device=self.device, dtype=dtype).contiguous()

        self.shared = get("shared.weight")
        self.layers = []
        for i in range(cfg.num_layers):
            a, m = f"encoder.block.{i}.layer.0.", f"encoder.block.{i}.layer.1."
            lay = {
                "ln0": get(a + "layer_norm.weight"),
                "wqkv": torch.cat([get(a + f"SelfAttention.{c}.weight") for c in "qkv"]),
                "wo_attn": get(a + "SelfAttention.o.weight"),
                "ln1": get(m + "layer_norm.weight"),
                "wi": torch.cat([get(m + "DenseReluDense.wi_0.weight"),
                                 get(m + "DenseReluDense.wi_1.weight")]),
                "wo": get(m + "DenseReluDense.wo.weight"),
            }
            if i == 0 or cfg.per_layer_bias:
                lay["rel"] = get(a + "SelfAttention.relative_attention_bias.weight")
            self.layers.append(lay)
        self.final_ln = get("encoder.final_layer_norm.weight")
        # the residual epilogue of the bf16 GEMM is residual + gate * (x W^T): a gate of ones
        self._ones = torch.ones(1, cfg.d_model, dtype=torch.bfloat16, device=self.device)
        self._buckets: dict[int, torch.Tensor] = {}

    # ------------------------------------------------------------------ pieces
    def buckets(self, s: int) -> torch.Tensor:
        b = self._buckets.get(s)
        if b is None:
            b = relative_position_buckets(s, s, self.cfg.relative_attention_num_buckets,
                                          self.cfg.relative_attention_max_distance).to(self.device)
            self._buckets[s] = b
        return b

    def _linear(self, x, w, out, residual=None):
        if self.dtype == torch.float32:
            kernels.gemm_f32(x, w, residual=residual, out=out)
            return
        if residual is None:
            p = kernels.Problem(x, w, out)
            epi = _lib.EPI_NONE
        else:
            p = kernels.Problem(x, w, out, gate=self._ones, residual=residual)
            epi = _lib.EPI_GATE_RESIDUAL
        kernels.gemm_grouped([p], kind="bf16", epilogue=epi, workspace="shared")

    def _attention(self, qkv, att, bias, b, s):
        cfg = self.cfg
        h, dk, inner = cfg.num_heads, cfg.d_kv, cfg.inner_dim
        view = lambda t, off, ld: t.as_strided((b, h, s, dk), (s * ld, dk, ld, 1),  # noqa: E731
                                               t.storage_offset() + off)
        q, k, v = (view(qkv, i * inner, 3 * inner) for i in range(3))
        kernels.attention(q, k, v, scale=1.0, attention_mask=bias, out=view(att, 0, inner))

    # ------------------------------------------------------------------ forward
    def forward(self, input_ids: torch.Tensor,
                attention_mask: torch.Tensor | None = None) -> torch.Tensor:
        cfg = self.cfg
        if input_ids.dim() != 2:
            raise ValueError("input_ids must be [batch, seq]")
        if attention_mask is not None and not cfg.per_layer_bias:
            # NeuronT5EncoderModel asserts the mask is None (modeling_t5.py:787)
            raise ValueError("the T5 encoder takes no attention mask (the prompt is encoded "
                             "whole, padding included)")
        b, s = input_ids.shape
        keep = None
        if attention_mask is not None:
            if tuple(attention_mask.shape) != (b, s):
                raise ValueError(f"attention_mask must be [{b}, {s}]")
            keep = (attention_mask.to(self.device) != 0).contiguous()
        dev, dt, rows = self.device, self.dtype, b * s
        x = kernels.embedding(input_ids.to(dev), self.shared).reshape(rows, cfg.d_model)
        if rows == 0:
            return x.reshape(b, s, cfg.d_model)
        qkv = torch.empty(rows, 3 * cfg.inner_dim, dtype=dt, device=dev)
        att = torch.empty(rows, cfg.inner_dim, dtype=dt, device=dev)
        ff = torch.empty(rows, 2 * cfg.d_ff, dtype=dt, device=dev)
        g = torch.empty(rows, cfg.d_ff, dtype=dt, device=dev)
        bias = None
        eps = cfg.layer_norm_epsilon
        for lay in self.layers:
            if "rel" in lay:
                bias = kernels.relative_bias(self.buckets(s), lay["rel"], batch=b if keep is not None else 1,
                                             seq_q=s, seq_k=s, key_keep=keep)
            n = kernels.rms_norm(x, lay["ln0"], eps)
            self._linear(n, lay["wqkv"], qkv)
            self._attention(qkv, att, bias, b, s)
            self._linear(att, lay["wo_attn"], x, residual=x)
            n = kernels.rms_norm(x, lay["ln1"], eps)
            self._linear(n, lay["wi"], ff)
            kernels.gated_gelu(ff, cfg.d_ff, out=g)
            self._linear(g, lay["wo"], x, residual=x)
        return kernels.rms_norm(x, self.final_ln, eps).reshape(b, s, cfg.d_model)

    __call__ = forward
