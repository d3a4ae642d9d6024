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
