"""Qwen-Image joint blocks and a reduced-depth Qwen-Image step on the HIP path against the fp32
oracle (bf16: rel L2 <= 1e-2; MXFP8 targets: the same-law and format-error checks the FLUX
tests explain)."""

import pytest
import torch

from difflet_amd import kernels
from difflet_amd.dit.qwen import QwenConfig, QwenImageDiT
from oracle import qwen as oqwen

pytestmark = pytest.mark.gpu

SEED = 4321
FORMAT_ERR = 6e-2


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _source(shape, n_blocks, seed=SEED):
    w = dict(oqwen.embed_weights(shape, seed))
    for i in range(n_blocks):
        for k, v in oqwen.block_weights(shape, seed, i).items():
            w[f"transformer_blocks.{i}.{k}"] = v
    return w


def _check_block(gpu, kind, st, img_hw, tol, parity):
    """One joint block: bf16 against the fp32 oracle; MX against the oracle of the same law
    with the device's bf16 rounding points and modulation vectors (see test_gpu_flux.py)."""
    print(f"qwen block {kind}, {st} + {img_hw[0] * img_hw[1]} tokens", flush=True)
    shape = oqwen.QwenShape(n_blocks=1)
    w = _source(shape, 1)
    dit = QwenImageDiT(QwenConfig(n_blocks=1), lambda n: w[n], kind=kind, device=gpu)
    g = torch.Generator().manual_seed(SEED)
    si = img_hw[0] * img_hw[1]
    hidden = torch.randn(1, si, shape.hidden, generator=g).bfloat16().float()
    context = torch.randn(1, st, shape.hidden, generator=g).bfloat16().float()
    temb = torch.randn(1, shape.hidden, generator=g).bfloat16().float()
    cos, sin = oqwen.pos_embed(img_hw[0], img_hw[1], st)
    bw = {k[len("transformer_blocks.0."):]: v for k, v in w.items()
          if k.startswith("transformer_blocks.0.")}
    bufs = dit._buffers(st, si)
    bufs["h"][:st] = context[0].to(gpu, torch.bfloat16)
    bufs["h"][st:] = hidden[0].to(gpu, torch.bfloat16)
    mod = kernels.gemv(temb.to(gpu, torch.bfloat16), dit.mod_w, dit.mod_b, act=1)
    gcos, gsin = dit.rope_tables(st, img_hw)
    dit.block(0, bufs, st, mod, gcos, gsin)
    torch.cuda.synchronize()
    out_c, out_h = bufs["h"][:st].float().cpu(), bufs["h"][st:].float().cpu()
    f_c, f_h = oqwen.block(bw, hidden, context, temb, cos, sin, shape)
    if kind == "bf16":
        e_c, e_h = rel_l2(out_c, f_c[0]), rel_l2(out_h, f_h[0])
        print(f"rel L2 vs fp32 oracle: text {e_c:.3e} image {e_h:.3e}", flush=True)
        parity("joint block, text rows, rel L2 vs fp32 oracle", e_c, tol)
        parity("joint block, image rows, rel L2 vs fp32 oracle", e_h, tol)
        assert e_c < tol and e_h < tol
        return
    d = shape.hidden
    mods = tuple(mod[:, dit.mod_off[(0, p)]:dit.mod_off[(0, p)] + 6 * d].float().cpu()
                 for p in ("img_mod", "txt_mod"))
    ref_c, ref_h = oqwen.block(bw, hidden, context, temb, cos, sin, shape, quant="mx",
                               act_dtype=torch.bfloat16, store=torch.bfloat16, mods=mods)
    e_c, e_h = rel_l2(out_c, ref_c[0]), rel_l2(out_h, ref_h[0])
    q_c, q_h = rel_l2(out_c, f_c[0]), rel_l2(out_h, f_h[0])
    o_c, o_h = rel_l2(ref_c, f_c), rel_l2(ref_h, f_h)
    print(f"rel L2 vs same-law oracle: text {e_c:.3e} image {e_h:.3e}; mx format error vs "
          f"fp32: device {q_c:.3e} / {q_h:.3e}, oracle {o_c:.3e} / {o_h:.3e}", flush=True)
    parity("joint block mx, text rows, rel L2 vs same-law oracle", e_c, tol)
    parity("joint block mx, image rows, rel L2 vs same-law oracle", e_h, tol)
    parity(f"joint block mx, image rows, format error vs fp32 (oracle's {o_h:.3e})", q_h,
           FORMAT_ERR)
    assert e_c < tol and e_h < tol
    assert abs(q_c - o_c) < 0.1 * o_c and abs(q_h - o_h) < 0.1 * o_h
    assert q_c < FORMAT_ERR and q_h < FORMAT_ERR


@pytest.mark.parametrize("kind,tol", [("bf16", 1e-2), ("mx", 3e-2)])
def test_qwen_block_matches_fp32_oracle(gpu, kind, tol, parity):
    st, img_hw = (256, (32, 32)) if kind == "bf16" else (128, (16, 16))
    _check_block(gpu, kind, st, img_hw, tol, parity)


def test_qwen_block_at_the_1328_step_shape_mx(gpu, parity):
    """The Qwen-Image 1328^2 step's own block shape: 256 text + 83 x 83 image tokens (7145
    rows, attention over 7145 keys on the split schedule), MXFP8 targets."""
    _check_block(gpu, "mx", 256, (83, 83), 3e-2, parity)


@pytest.mark.parametrize("kind,tol", [("bf16", 1e-2), ("mx", 3e-2)])
def test_qwen_reduced_depth_step_matches_fp32_oracle(gpu, kind, tol, parity):
    """img_in, txt_norm + txt_in, the timestep embedder, 2 joint blocks and norm_out / proj_out
    at Qwen-Image width on an odd 15 x 17 patch grid (centred RoPE positions) + 64 text tokens."""
    print(f"qwen reduced step {kind}", flush=True)
    shape = oqwen.QwenShape(n_blocks=2)
    w = _source(shape, 2)
    img_hw, st = (15, 17), 64
    inp = oqwen.synthetic_inputs(shape, SEED, img_hw, st)
    lat, txt = inp["latents"].bfloat16().float(), inp["text"].bfloat16().float()
    quant = "mx" if kind == "mx" else None
    ref = oqwen.forward(shape, SEED, lat, txt, inp["timestep"], img_hw,
                        weights=(oqwen.embed_weights(shape, SEED),
                                 [oqwen.block_weights(shape, SEED, i) for i in range(2)]),
                        model_dtype=torch.bfloat16, quant=quant,
                        act_dtype=torch.bfloat16 if quant else None,
                        store=torch.bfloat16 if quant else None)
    dit = QwenImageDiT(QwenConfig(n_blocks=2), lambda n: w[n], kind=kind, device=gpu)
    out = dit.forward(lat.to(gpu), txt.to(gpu), inp["timestep"].to(gpu), img_hw)
    torch.cuda.synchronize()
    e = rel_l2(out, ref)
    print(f"step rel L2 {e:.3e}", flush=True)
    parity(f"2-block step {kind}, rel L2 vs {'same-law' if quant else 'fp32'} oracle", e, tol)
    assert out.shape == (1, 255, 64)
    assert e < tol


@pytest.mark.parametrize("valid", [40, 0])
def test_qwen_padded_prompt_matches_the_masked_oracle(gpu, valid, parity):
    """A prompt right-padded to 64 rows with `valid` real ones: the step with text_valid_len
    against the oracle running the reference's masked joint attention (text keys from `valid`
    on masked in every block, modeling_qwen_image.py:493-552) over the padded prompt."""
    print(f"qwen padded prompt, valid {valid} of 64", flush=True)
    shape = oqwen.QwenShape(n_blocks=2)
    w = _source(shape, 2)
    img_hw, st = (15, 17), 64
    inp = oqwen.synthetic_inputs(shape, SEED, img_hw, st)
    lat, txt = inp["latents"].bfloat16().float(), inp["text"].bfloat16().float()
    weights = (oqwen.embed_weights(shape, SEED), [oqwen.block_weights(shape, SEED, i)
                                                  for i in range(2)])
    ref = oqwen.forward(shape, SEED, lat, txt, inp["timestep"], img_hw, weights=weights,
                        model_dtype=torch.bfloat16, text_valid_len=valid)
    unmasked = oqwen.forward(shape, SEED, lat, txt, inp["timestep"], img_hw, weights=weights,
                             model_dtype=torch.bfloat16)
    dit = QwenImageDiT(QwenConfig(n_blocks=2), lambda n: w[n], kind="bf16", device=gpu)
    out = dit.forward(lat.to(gpu), txt.to(gpu), inp["timestep"].to(gpu), img_hw,
                      text_valid_len=torch.tensor([valid], dtype=torch.int32))
    torch.cuda.synchronize()
    e, gap = rel_l2(out, ref), rel_l2(unmasked, ref)
    print(f"padded step rel L2 vs masked oracle {e:.3e} (masking moves the oracle {gap:.3e})",
          flush=True)
    parity(f"padded prompt ({valid} of 64 rows), rel L2 vs masked fp32 oracle", e, 1e-2)
    assert out.shape == (1, 255, 64)
    assert e < 1e-2 and gap > 2 * e

