"""The Qwen-Image oracle: block invariants, the RoPE table's closed form and the MXFP8 target
list."""

import re

import torch

from oracle import ops
from oracle import qwen as oqwen

SMALL = oqwen.QwenShape(hidden=256, heads=2, head_dim=128, mlp=512, n_blocks=1, txt_dim=96)


def _inputs(seed=0, st=5, si=7):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(1, si, SMALL.hidden, generator=g), torch.randn(1, st, SMALL.hidden, generator=g),
            torch.randn(1, SMALL.hidden, generator=g))


def test_zero_gates_make_the_block_the_identity():
    w = oqwen.block_weights(SMALL, 3, 0, dtype=torch.float32)
    d = SMALL.hidden
    for part in ("img_mod.1", "txt_mod.1"):
        # gates are chunks 2 and 5 of the 6 modulation vectors
        for c in (2, 5):
            w[f"{part}.weight"][c * d:(c + 1) * d] = 0
            w[f"{part}.bias"][c * d:(c + 1) * d] = 0
    hidden, context, temb = _inputs()
    cos, sin = oqwen.pos_embed(1, 7, 5)
    c2, h2 = oqwen.block(w, hidden, context, temb, cos, sin, SMALL)
    assert torch.equal(c2, context) and torch.equal(h2, hidden)


def test_block_attention_is_one_joint_softmax_text_first():
    """With identity modulation, unit gates and zero MLPs the block adds to_out(attention) of the
    joint [text | image] sequence: recompute that attention directly."""
    w = oqwen.block_weights(SMALL, 5, 0, dtype=torch.float32)
    d = SMALL.hidden
    for part in ("img_mod.1", "txt_mod.1"):
        w[f"{part}.weight"].zero_()
        b = torch.zeros(6 * d)
        b[2 * d:3 * d] = 1.0  # gate 1 = 1, shifts / scales / gate 2 = 0
        w[f"{part}.bias"] = b
    hidden, context, temb = _inputs(1)
    cos, sin = oqwen.pos_embed(1, 7, 5)
    c2, h2 = oqwen.block(w, hidden, context, temb, cos, sin, SMALL)
    L = ops.linear
    nx, nc = ops.layer_norm(hidden), ops.layer_norm(context)
    heads = lambda x: x.view(1, -1, 2, 128).transpose(1, 2)  # noqa: E731
    qkv = lambda x, fmt: [heads(L(x, w[f"attn.{fmt % n}.weight"], w[f"attn.{fmt % n}.bias"]))  # noqa: E731
                          for n in ("q", "k", "v")]
    q, k, v = qkv(nx, "to_%s")
    cq, ck, cv = qkv(nc, "add_%s_proj")
    cq, ck = (ops.rms_norm_fp32(t, torch.ones(128), 1e-6) for t in (cq, ck))
    q, k = (ops.rms_norm_fp32(t, torch.ones(128), 1e-6) for t in (q, k))
    qj = ops.apply_rotary_emb_fp32(torch.cat([cq, q], 2), cos[None, None], sin[None, None])
    kj = ops.apply_rotary_emb_fp32(torch.cat([ck, k], 2), cos[None, None], sin[None, None])
    p = torch.softmax(qj @ kj.transpose(-1, -2) / 128 ** 0.5, dim=-1)
    o = (p @ torch.cat([cv, v], 2)).transpose(1, 2).reshape(1, 12, d)
    ref_h = hidden + L(o[:, 5:], w["attn.to_out.0.weight"], w["attn.to_out.0.bias"])
    ref_c = context + L(o[:, :5], w["attn.to_add_out.weight"], w["attn.to_add_out.bias"])
    # the MLP still adds gate 2 (zero) * mlp: exactly the attention residual remains
    assert torch.allclose(h2, ref_h, atol=1e-5) and torch.allclose(c2, ref_c, atol=1e-5)


def test_rope_table_closed_form():
    h, w, st = 5, 4, 3
    cos, sin = oqwen.pos_embed(h, w, st)
    assert cos.shape == (st + h * w, 128)
    inv = lambda dim: 1.0 / 10000.0 ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim)  # noqa: E731
    # text token j sits at max(h // 2, w // 2) + j on all three axes
    for j in range(st):
        pos = max(h // 2, w // 2) + j
        ang = torch.cat([pos * inv(16), pos * inv(56), pos * inv(56)])
        assert torch.allclose(cos[j, 0::2].double(), torch.cos(ang), atol=1e-5)
        assert torch.allclose(sin[j, 1::2].double(), torch.sin(ang), atol=1e-5)
    # image patch (y, x): frame 0, height y - (h - h // 2), width x - (w - w // 2)
    for y in range(h):
        for x in range(w):
            r = st + y * w + x
            ang = torch.cat([0 * inv(16), (y - (h - h // 2)) * inv(56), (x - (w - w // 2)) * inv(56)])
            assert torch.allclose(cos[r, 0::2].double(), torch.cos(ang), atol=1e-5)
            assert torch.allclose(sin[r, 0::2].double(), torch.sin(ang), atol=1e-5)
    # pairs share an angle (interleaved law)
    assert torch.equal(cos[:, 0::2], cos[:, 1::2]) and torch.equal(sin[:, 0::2], sin[:, 1::2])


def test_device_rope_tables_equal_the_oracle():
    from difflet_amd.dit.rope import qwen_rope_tables

    for h, w, st in ((83, 83, 256), (15, 17, 64)):
        c0, s0 = oqwen.pos_embed(h, w, st)
        c1, s1 = qwen_rope_tables(st, (h, w), device="cpu")
        assert torch.equal(c0, c1) and torch.equal(s0, s1)


def test_mx_targets_are_the_qwen_image_targets():
    from difflet_amd.quant.spec import QWEN_IMAGE_TARGETS

    match = lambda n: any(re.fullmatch(p, n) for p in QWEN_IMAGE_TARGETS)  # noqa: E731
    names = {k.rsplit(".", 1)[0] for k, _ in oqwen.block_params(SMALL) if k.endswith(".weight")}
    for n in names:
        assert match(f"transformer_blocks.7.{n}") == (n in oqwen.MX_TARGETS), n


# ------------------------------------------------ unit gates: a plain transformer block
def _unit_gate_weights(seed):
    """Zero modulation weights, biases that give shift = scale = 0 and gate = 1 on both
    streams; random q/k norm weights so the norm's affine step is exercised too."""
    w = oqwen.block_weights(SMALL, seed, 0, dtype=torch.float32)
    d = SMALL.hidden
    for part in ("img_mod.1", "txt_mod.1"):
        w[f"{part}.weight"].zero_()
        b = torch.zeros(6 * d)
        b[2 * d:3 * d] = 1.0  # gate 1
        b[5 * d:6 * d] = 1.0  # gate 2
        w[f"{part}.bias"] = b
    g = torch.Generator().manual_seed(seed)
    for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
        w[f"attn.{n}.weight"] = 0.5 + torch.rand(128, generator=g)
    return w


def _plain_qwen_block(w, x, c, cos, sin):
    """Pre-LN joint block from torch primitives: F.layer_norm, F.rms_norm, RoPE as complex
    multiplication, F.scaled_dot_product_attention over [text | image], F.gelu(tanh) MLPs."""
    import torch.nn.functional as F

    d, st = SMALL.hidden, c.shape[1]
    heads = lambda t: t.view(1, -1, 2, 128).transpose(1, 2)  # noqa: E731
    lin = lambda t, n: F.linear(t, w[f"{n}.weight"], w[f"{n}.bias"])  # noqa: E731
    ln = lambda t: F.layer_norm(t, (d,), eps=1e-6)  # noqa: E731
    rms = lambda t, n: F.rms_norm(t, (128,), w[f"attn.{n}.weight"], 1e-6)  # noqa: E731
    ang = torch.atan2(sin[:, 0::2], cos[:, 0::2])

    def rope(t):
        z = torch.view_as_complex(t.reshape(*t.shape[:-1], 64, 2).contiguous())
        return torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)).reshape(t.shape)

    nx, nc = ln(x), ln(c)
    q = torch.cat([rms(heads(lin(nc, "attn.add_q_proj")), "norm_added_q"),
                   rms(heads(lin(nx, "attn.to_q")), "norm_q")], dim=2)
    k = torch.cat([rms(heads(lin(nc, "attn.add_k_proj")), "norm_added_k"),
                   rms(heads(lin(nx, "attn.to_k")), "norm_k")], dim=2)
    v = torch.cat([heads(lin(nc, "attn.add_v_proj")), heads(lin(nx, "attn.to_v"))], dim=2)
    o = F.scaled_dot_product_attention(rope(q), rope(k), v).transpose(1, 2).reshape(1, -1, d)
    x = x + lin(o[:, st:], "attn.to_out.0")
    c = c + lin(o[:, :st], "attn.to_add_out")
    mlp = lambda t, s: lin(F.gelu(lin(ln(t), f"{s}.net.0.proj"), approximate="tanh"), f"{s}.net.2")  # noqa: E731
    return c + mlp(c, "txt_mlp"), x + mlp(x, "img_mlp")


def _unit_gate_case(seed=11):
    w = _unit_gate_weights(seed)
    hidden, context, temb = _inputs(seed)
    cos, sin = oqwen.pos_embed(1, 7, 5)
    return w, hidden, context, temb, cos, sin


def test_unit_gates_make_the_block_a_plain_transformer_block():
    """Zero shift / scale and unit gates reduce the block (attention and both MLPs) to a plain
    pre-LN joint transformer block computed from torch's own primitives."""
    w, hidden, context, temb, cos, sin = _unit_gate_case()
    c_ref, h_ref = _plain_qwen_block(w, hidden, context, cos, sin)
    c2, h2 = oqwen.block(w, hidden, context, temb, cos, sin, SMALL)
    assert torch.allclose(h2, h_ref, atol=1e-5, rtol=1e-5)
    assert torch.allclose(c2, c_ref, atol=1e-5, rtol=1e-5)


def test_planted_exact_gelu_is_seen_by_the_plain_block(monkeypatch):
    """The unit-gate check fails an oracle whose MLP takes the exact GELU."""
    w, hidden, context, temb, cos, sin = _unit_gate_case()
    c_ref, h_ref = _plain_qwen_block(w, hidden, context, cos, sin)
    monkeypatch.setattr(ops, "gelu_tanh", lambda x: torch.nn.functional.gelu(x))
    c2, h2 = oqwen.block(w, hidden, context, temb, cos, sin, SMALL)
    assert not torch.allclose(h2, h_ref, atol=1e-5, rtol=1e-5)
    assert not torch.allclose(c2, c_ref, atol=1e-5, rtol=1e-5)


def test_planted_swapped_chunk_order_is_seen_by_the_plain_block():
    """Modulation vectors read in another chunk order (scale where the gate belongs) fail the
    unit-gate check: the block then scales LN(x) by 2 and closes both gates."""
    w, hidden, context, temb, cos, sin = _unit_gate_case()
    c_ref, h_ref = _plain_qwen_block(w, hidden, context, cos, sin)
    d = SMALL.hidden
    silu = torch.nn.functional.silu(temb)
    mods = [ops.linear(silu, w[f"{p}.weight"], w[f"{p}.bias"]) for p in ("img_mod.1", "txt_mod.1")]
    swapped = [torch.cat([m[:, :d], m[:, 2 * d:3 * d], m[:, d:2 * d], m[:, 3 * d:]], dim=1)
               for m in mods]
    c2, h2 = oqwen.block(w, hidden, context, temb, cos, sin, SMALL, mods=tuple(swapped))
    assert not torch.allclose(h2, h_ref, atol=1e-3)
    # the vectors in their own order reproduce the check
    c3, h3 = oqwen.block(w, hidden, context, temb, cos, sin, SMALL, mods=tuple(mods))
    assert torch.allclose(h3, h_ref, atol=1e-5, rtol=1e-5)


def test_masked_text_keys_equal_the_trimmed_prompt():
    """The reference's masked joint attention (keys [image | text] bounded at S_img + valid)
    gives the image stream, and the valid text rows, that the prompt cut to its valid rows
    gives: masked keys take no weight and padded queries influence nothing."""
    w = oqwen.block_weights(SMALL, 13, 0, dtype=torch.float32)
    hidden, context, temb = _inputs(13, st=9)
    cos, sin = oqwen.pos_embed(1, 7, 9)
    valid = 4
    c_m, h_m = oqwen.block(w, hidden, context, temb, cos, sin, SMALL, text_valid_len=valid)
    cos_t = torch.cat([cos[:valid], cos[9:]])
    sin_t = torch.cat([sin[:valid], sin[9:]])
    c_t, h_t = oqwen.block(w, hidden, context[:, :valid], temb, cos_t, sin_t, SMALL)
    assert torch.allclose(h_m, h_t, atol=1e-5, rtol=1e-5)
    assert torch.allclose(c_m[:, :valid], c_t, atol=1e-5, rtol=1e-5)
    # and it differs from attending to the padding
    _, h_u = oqwen.block(w, hidden, context, temb, cos, sin, SMALL)
    assert not torch.allclose(h_u, h_m, atol=1e-3)
    # a fully valid prompt is the unmasked block
    _, h_f = oqwen.block(w, hidden, context, temb, cos, sin, SMALL, text_valid_len=9)
    assert torch.allclose(h_f, h_u, atol=1e-5, rtol=1e-5)


# ------------------------------------- step level: time embedding, text embedding, final layer
# The model-level functions reduced to torch primitives and closed forms (identity linears,
# distinct scale / shift vectors), each paired with a planted mistake that fails it. The laws:
# diffusers' QwenTimestepProjEmbeddings (the model casts t / 1000 to its dtype, the sinusoid of
# 256 channels, cos first, shift 0, scales its argument by 1000), txt_norm = RMSNorm (eps 1e-6)
# before txt_in, and AdaLN-Continuous (difflet/layers/normalization.py:150-190: emb =
# linear(SiLU(temb)), chunk scale first, LayerNorm without affine).
STEP = oqwen.QwenShape(hidden=256, heads=2, head_dim=128, mlp=512, n_blocks=0,
                       in_channels=256, out_channels=256, txt_dim=256)
T_FRAC = torch.tensor([0.0, 0.7137, 0.4219])  # t / 1000; 1000 * bf16(0.7137) is not a bf16 value


def _sinusoid64(arg, dim=256):
    """cos / sin halves of exp(-ln(10000) i / 128) * arg, i < 128, in float64."""
    import math

    import numpy as np

    half = dim // 2
    f = np.exp(-math.log(10000.0) * np.arange(half) / half)
    a = np.outer(np.asarray(arg, dtype=np.float64), f)
    return torch.from_numpy(np.concatenate([np.cos(a), np.sin(a)], axis=1))


def _identity_embedders(seed=8):
    d = STEP.hidden
    ew = oqwen.embed_weights(STEP, seed, dtype=torch.float32)
    te = "time_text_embed.timestep_embedder."
    for n in ("linear_1", "linear_2"):
        ew[f"{te}{n}.weight"], ew[f"{te}{n}.bias"] = torch.eye(d), torch.zeros(d)
    ew["txt_in.weight"], ew["txt_in.bias"] = torch.eye(d), torch.zeros(d)
    ew["img_in.weight"], ew["img_in.bias"] = torch.eye(d), torch.zeros(d)
    ew["proj_out.weight"], ew["proj_out.bias"] = torch.eye(d), torch.zeros(d)
    g = torch.Generator().manual_seed(seed)
    ew["txt_norm.weight"] = 0.5 + torch.rand(d, generator=g)
    return ew


def _check_time_embed(ew, model_dtype):
    """time_embed with identity linears is silu(sinusoid(1000 * t')), t' = t / 1000 in the model
    dtype."""
    import torch.nn.functional as F

    temb = oqwen.time_embed(ew, T_FRAC, model_dtype)
    arg = T_FRAC.to(model_dtype).double() * 1000.0
    return torch.allclose(temb.double(), F.silu(_sinusoid64(arg)), atol=3e-4, rtol=0)


def test_time_embed_reduces_to_silu_of_the_sinusoid_of_1000_t():
    ew = _identity_embedders()
    assert _check_time_embed(ew, torch.float32)
    assert _check_time_embed(ew, torch.bfloat16)
    temb = oqwen.time_embed(ew, torch.zeros(1))  # t = 0: cos 0 = 1, sin 0 = 0
    assert torch.allclose(temb[0, :128], torch.nn.functional.silu(torch.ones(128)))
    assert torch.equal(temb[0, 128:], torch.zeros(128))


def test_planted_timestep_cast_after_the_1000_scale_is_seen(monkeypatch):
    """Rounding 1000 t' to bf16 (a cast after the scale, not of t / 1000 before it) fails."""
    ew = _identity_embedders()
    real = ops.timestep_embedding
    monkeypatch.setattr(ops, "timestep_embedding",
                        lambda t, dim, **kw: real(t.to(torch.bfloat16).float(), dim, **kw))
    assert not _check_time_embed(ew, torch.bfloat16)


def test_planted_sin_first_time_embedding_is_seen(monkeypatch):
    ew = _identity_embedders()
    real = ops.timestep_embedding
    monkeypatch.setattr(ops, "timestep_embedding",
                        lambda t, dim, **kw: real(t, dim, **{**kw, "flip_sin_to_cos": False}))
    assert not _check_time_embed(ew, torch.float32)


def _text_case(seed=9):
    return torch.randn(1, 6, STEP.txt_dim, generator=torch.Generator().manual_seed(seed)) * 3 + 1


def test_text_embedding_is_rms_norm_then_txt_in():
    ew = _identity_embedders()
    text = _text_case()
    ref = torch.nn.functional.rms_norm(text, (STEP.txt_dim,), ew["txt_norm.weight"], 1e-6)
    assert torch.allclose(oqwen.embed_text(ew, text), ref, atol=1e-5, rtol=1e-5)


def test_planted_layer_norm_for_txt_norm_is_seen(monkeypatch):
    """A LayerNorm (mean removed) in place of the RMSNorm fails the check."""
    ew = _identity_embedders()
    text = _text_case()
    ref = torch.nn.functional.rms_norm(text, (STEP.txt_dim,), ew["txt_norm.weight"], 1e-6)
    monkeypatch.setattr(ops, "rms_norm_fp32", lambda x, w, eps: torch.nn.functional.layer_norm(
        x, (x.shape[-1],), w, None, eps))
    assert not torch.allclose(oqwen.embed_text(ew, text), ref, atol=1e-3)


def _final_case(seed=10):
    d = STEP.hidden
    ew = _identity_embedders(seed)
    g = torch.Generator().manual_seed(seed)
    a, b = 0.75, -1.25
    ew["norm_out.linear.weight"] = torch.cat([a * torch.eye(d), b * torch.eye(d)])
    ew["norm_out.linear.bias"] = torch.randn(2 * d, generator=g)
    hidden = torch.randn(1, 9, d, generator=g) * 2 - 0.5
    temb = torch.randn(1, d, generator=g)
    silu = torch.nn.functional.silu(temb)
    scale = a * silu + ew["norm_out.linear.bias"][:d]
    shift = b * silu + ew["norm_out.linear.bias"][d:]
    ref = torch.nn.functional.layer_norm(hidden, (d,), eps=1e-6) * (1 + scale[:, None]) \
        + shift[:, None]
    return ew, hidden, temb, ref


def test_final_layer_is_ada_layer_norm_continuous_scale_first():
    ew, hidden, temb, ref = _final_case()
    assert torch.allclose(oqwen.final_layer(ew, hidden, temb), ref, atol=1e-5, rtol=1e-5)


def test_planted_shift_first_final_layer_is_seen():
    """An oracle reading the AdaLN-Continuous chunks as (shift, scale) fails the check: the
    same as this oracle with the two halves of the linear exchanged."""
    ew, hidden, temb, ref = _final_case()
    d = STEP.hidden
    swapped = dict(ew)
    for n in ("weight", "bias"):
        t = ew[f"norm_out.linear.{n}"]
        swapped[f"norm_out.linear.{n}"] = torch.cat([t[d:], t[:d]])
    assert not torch.allclose(oqwen.final_layer(swapped, hidden, temb), ref, atol=1e-3)


def test_step_without_blocks_is_img_in_then_the_final_layer():
    """forward() with no blocks: img_in, the time embedding of t / 1000, the final layer (the
    text path and the RoPE table are built and unused)."""
    ew, _, _, _ = _final_case(11)
    g = torch.Generator().manual_seed(12)
    lat = torch.randn(1, 12, STEP.in_channels, generator=g)
    text = _text_case(13)
    t = torch.tensor([0.4219])
    out = oqwen.forward(STEP, 0, lat, text, t, (3, 4), weights=(ew, []))
    temb = oqwen.time_embed(ew, t)
    d = STEP.hidden
    emb = torch.nn.functional.silu(temb) @ ew["norm_out.linear.weight"].T + ew["norm_out.linear.bias"]
    ref = torch.nn.functional.layer_norm(lat, (d,), eps=1e-6) * (1 + emb[:, None, :d]) \
        + emb[:, None, d:]
    assert torch.allclose(out, ref, atol=1e-5, rtol=1e-5)
