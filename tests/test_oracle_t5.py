"""Pins of the T5 / UMT5 encoder oracle (oracle/t5.py).

The reference's T5 is transformers' T5 encoder forked module for module (modeling_t5.py:15-20)
and its UMT5 mirrors transformers' UMT5EncoderModel key for key (modeling_umt5.py:1-16), so the
installed transformers (5.15.0) encoders, built from the same weights, are the independent
check: whole stacks in fp32, with and without a padding mask. The bucket function is also
checked against values worked out by hand from its definition. Each pin is paired with a
planted mistake (in the oracle, on the CPU) that it must catch.
"""

import dataclasses

import pytest
import torch

from oracle import t5 as ot5

SMALL = ot5.T5Shape(vocab=300, d_model=128, d_kv=32, d_ff=256, heads=4, layers=3)
SMALL_UMT5 = dataclasses.replace(SMALL, per_layer_bias=True)
SEQ = 150  # past max_distance (128): every bucket, the clamped last one included, is used
TOL = 1e-6  # measured: 0 (bit-identical) on both stacks


def rel_l2(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def _hf(shape: ot5.T5Shape, w):
    tr = pytest.importorskip("transformers")
    kw = dict(vocab_size=shape.vocab, d_model=shape.d_model, d_kv=shape.d_kv, d_ff=shape.d_ff,
              num_layers=shape.layers, num_heads=shape.heads,
              relative_attention_num_buckets=shape.buckets,
              relative_attention_max_distance=shape.max_distance,
              layer_norm_epsilon=shape.eps, feed_forward_proj="gated-gelu", dropout_rate=0.0)
    if shape.per_layer_bias:
        model = tr.UMT5EncoderModel(tr.UMT5Config(**kw))
    else:
        model = tr.T5EncoderModel(tr.T5Config(**kw))
    sd = dict(w)
    sd["encoder.embed_tokens.weight"] = w["shared.weight"]
    model.load_state_dict(sd, strict=True)
    return model.eval()


def _ids(b, s, vocab, seed=3):
    return torch.randint(0, vocab, (b, s), generator=torch.Generator().manual_seed(seed))


def test_bucket_values_worked_by_hand():
    """32 buckets, max_distance 128: 16 per direction, distances 0..7 exact, then
    8 + floor(log(d / 8) / log(16) * 8), at most 15; keys after the query add 16."""
    rel = torch.tensor([0, -1, -7, 1, 7, -8, 8, -12, -20, -100, -127, -128, -1000, 1000, 50, 12])
    want = [0, 1, 7, 17, 23, 8, 24, 9, 10, 15, 15, 15, 15, 31, 29, 25]
    # -12: 8 + floor(8 ln 1.5 / ln 16) = 8 + floor(1.17); -20: 8 + floor(2.64); -100: 8 +
    # floor(7.29); -127: 8 + floor(7.98); -128 and beyond: min(16, 15); +50: 16 + 8 + floor(5.29)
    assert ot5.relative_position_bucket(rel, 32, 128).tolist() == want


def test_buckets_equal_transformers_and_are_monotone():
    tr = pytest.importorskip("transformers.models.t5.modeling_t5")
    rel = torch.arange(-700, 701)[None, :]
    ours = ot5.relative_position_bucket(rel, 32, 128)
    lib = tr.T5Attention._relative_position_bucket(rel, bidirectional=True, num_buckets=32,
                                                   max_distance=128)
    assert torch.equal(ours, lib)
    neg, pos = ours[0, :701].flip(0), ours[0, 700:]
    assert (neg.diff() >= 0).all() and (pos[1:].diff() >= 0).all()
    assert set(ours.unique().tolist()) == set(range(32)) - {16}


@pytest.mark.parametrize("shape", [SMALL, SMALL_UMT5], ids=["t5", "umt5"])
def test_encoder_equals_transformers(shape):
    w = ot5.weights(shape, 5)
    ids = _ids(2, SEQ, shape.vocab)
    ref = _hf(shape, w)(input_ids=ids).last_hidden_state
    out = ot5.encode(w, shape, ids)
    assert rel_l2(out, ref) < TOL


def test_umt5_padding_mask_equals_transformers():
    w = ot5.weights(SMALL_UMT5, 6)
    ids = _ids(2, SEQ, SMALL_UMT5.vocab, seed=4)
    mask = torch.ones(2, SEQ, dtype=torch.long)
    mask[1, 97:] = 0
    ref = _hf(SMALL_UMT5, w)(input_ids=ids, attention_mask=mask).last_hidden_state
    out = ot5.encode(w, SMALL_UMT5, ids, attention_mask=mask)
    assert rel_l2(out, ref) < TOL
    # the padding changes the padded prompt's real tokens, and only that prompt
    free = ot5.encode(w, SMALL_UMT5, ids)
    assert rel_l2(out[1, :97], free[1, :97]) > 1e-3
    assert rel_l2(out[0], free[0]) < 1e-7


def test_t5_refuses_a_mask():
    with pytest.raises(ValueError, match="no attention mask"):
        ot5.encode(ot5.weights(SMALL, 1), SMALL, _ids(1, 4, SMALL.vocab), torch.ones(1, 4))


# ------------------------------------------------------------------- planted mistakes
def _err_vs_hf(shape, monkeypatch, name, fn, mask=False):
    w = ot5.weights(shape, 5)
    ids = _ids(2, SEQ, shape.vocab)
    am = None
    if mask:
        am = torch.ones(2, SEQ, dtype=torch.long)
        am[1, 97:] = 0
    ref = _hf(shape, w)(input_ids=ids, attention_mask=am).last_hidden_state
    if name is not None:
        monkeypatch.setattr(ot5, name, fn)
    return rel_l2(ot5.encode(w, shape, ids, attention_mask=am), ref)


def test_planted_exact_gelu_is_caught(monkeypatch):
    e = _err_vs_hf(SMALL, monkeypatch, "gelu_new", torch.nn.functional.gelu)
    assert e > 20 * TOL


def test_planted_bucket_direction_is_caught(monkeypatch):
    real = ot5.relative_position_bucket
    e = _err_vs_hf(SMALL, monkeypatch, "relative_position_bucket",
                   lambda rel, nb, md: real(-rel, nb, md))
    assert e > 20 * TOL


def test_planted_bucket_off_by_one_is_caught(monkeypatch):
    real = ot5.relative_position_bucket
    e = _err_vs_hf(SMALL_UMT5, monkeypatch, "relative_position_bucket",
                   lambda rel, nb, md: real(rel + 1, nb, md))
    assert e > 20 * TOL


def test_planted_unweighted_norm_is_caught(monkeypatch):
    real = ot5.rms_norm
    e = _err_vs_hf(SMALL, monkeypatch, "rms_norm", lambda x, w, eps: real(x, torch.ones_like(w), eps))
    assert e > 20 * TOL


def test_planted_shared_bias_in_umt5_is_caught():
    """UMT5 with block 0's table reused everywhere (the T5 rule) differs from transformers."""
    w = ot5.weights(SMALL_UMT5, 5)
    ids = _ids(2, SEQ, SMALL_UMT5.vocab)
    ref = _hf(SMALL_UMT5, w)(input_ids=ids).last_hidden_state
    shared = dataclasses.replace(SMALL_UMT5, per_layer_bias=False)
    assert rel_l2(ot5.encode(w, shared, ids), ref) > 20 * TOL


def test_planted_ignored_padding_is_caught(monkeypatch):
    e = _err_vs_hf(SMALL_UMT5, monkeypatch, "padding_mask",
                   lambda m: torch.zeros(m.shape[0], 1, 1, m.shape[1]), mask=True)
    assert e > 20 * TOL


def test_store_rounding_moves_the_result_by_bf16_steps():
    """The bf16 rounding points move the output by about bf16 precision and no more."""
    w = ot5.weights(SMALL, 7, torch.bfloat16)
    ids = _ids(1, 64, SMALL.vocab)
    e = rel_l2(ot5.encode(w, SMALL, ids, store=torch.bfloat16), ot5.encode(w, SMALL, ids))
    assert 1e-4 < e < 2e-2
