"""FLUX blocks and a reduced-depth FLUX step on the HIP path against the fp32 oracle.

Tolerances are the north-star's: relative L2 <= 1e-2 for bf16 and <= 3e-2 for the fp8 /
MXFP8 linears, each against the unquantized fp32 CPU computation on the same (bf16-rounded)
weights and inputs.
"""

import pytest
import torch

from difflet_amd import kernels
from difflet_amd.dit.flux import FluxConfig, FluxDiT
from oracle import flux as oflux
from oracle import ops

pytestmark = pytest.mark.gpu

SEED = 1234


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _source(shape, n_double, n_single, seed=SEED):
    """Oracle weights under the diffusers names FluxDiT reads."""
    w = {}
    for k, v in oflux.embed_weights(shape, seed).items():
        w[k] = v
    for i in range(n_double):
        for k, v in oflux.double_block_weights(shape, seed, i).items():
            w[f"transformer_blocks.{i}.{k}"] = v
    for i in range(n_single):
        for k, v in oflux.single_block_weights(shape, seed, i).items():
            w[f"single_transformer_blocks.{i}.{k}"] = v
    return w


def _block_setup(gpu, kind, st=None, img_hw=None):
    # config 1's shape (512 text + 32 x 32 image tokens) for bf16; the quantized cases use
    # 256 + 16 x 16 tokens so the CPU run of the quantization laws stays short
    st = st or (512 if kind == "bf16" else 256)
    img_hw = img_hw or ((32, 32) if kind == "bf16" else (16, 16))
    shape = oflux.FluxShape(n_double=1, n_single=1)
    cfg = FluxConfig(n_double=1, n_single=1)
    w = _source(shape, 1, 1)
    dit = FluxDiT(cfg, lambda n: w[n], kind=kind, device=gpu)
    g = torch.Generator().manual_seed(SEED)
    si = img_hw[0] * img_hw[1]
    hidden = torch.randn(1, si, shape.hidden, generator=g).bfloat16().float()
    context = torch.randn(1, st, shape.hidden, generator=g).bfloat16().float()
    temb = torch.randn(1, shape.hidden, generator=g).bfloat16().float()
    return shape, w, dit, hidden, context, temb, st, img_hw


def _gpu_mod(dit, temb, gpu):
    """Every block's adaLN vectors: linear(silu(temb)) through the GEMV kernel."""
    return kernels.gemv(temb.to(gpu, torch.bfloat16), dit.mod_w, dit.mod_b, act=1)


def _host_mods(dit, mod, key, n):
    """The device's bf16 modulation vectors of one adaLN (n chunks of D) as fp32 on the host."""
    off, d = dit.mod_off[key], dit.cfg.hidden
    return mod[:, off:off + n * d].float().cpu()


# bf16: the device against the fp32 oracle, rel L2 <= 1e-2.
# fp8 / mx: the device against the oracle of the same quantization law, rel L2 <= 3e-2. That
# oracle rounds to bf16 wherever the device stores bf16 and takes the device's bf16 modulation
# vectors, so both quantize the same activations: a value that lands on the other side of an
# e4m3 rounding midpoint moves by 1/16 of itself, and inputs that differ by bf16 rounding flip
# enough such bins to cost ~3e-2 on their own. Second check: the device's error against the
# unquantized fp32 block equals the oracle's own (the format's error) within 10 %; a wrong
# scale, block or rounding rule moves it far more. That format error is the e4m3 format's own,
# ~4.8e-2 at FLUX width on these N(0, 0.02) weights (measured on the oracle alone).
CASES = [("bf16", None), ("fp8", "fp8"), ("mx", "mx")]
TOL = {"bf16": 1e-2, "fp8": 3e-2, "mx": 3e-2}
FORMAT_ERR = 6e-2


def _check_double(gpu, kind, quant, parity, st=None, img_hw=None):
    shape, w, dit, hidden, context, temb, st, img_hw = _block_setup(gpu, kind, st, img_hw)
    print(f"flux double block {kind}, {st} + {img_hw[0] * img_hw[1]} tokens", flush=True)
    cos, sin = ops.flux_pos_embed(ops.flux_ids(st, *img_hw))
    bw = {k[len("transformer_blocks.0."):]: v for k, v in w.items()
          if k.startswith("transformer_blocks.0.")}
    bufs = dit._buffers(st, hidden.shape[1])
    bufs["h"][:st] = context[0].to(gpu, torch.bfloat16)
    bufs["h"][st:] = hidden[0].to(gpu, torch.bfloat16)
    mod = _gpu_mod(dit, temb, gpu)
    gcos, gsin = dit.rope_tables(st, img_hw)
    dit.double_block(0, bufs, st, mod, gcos, gsin)
    torch.cuda.synchronize()
    out_c, out_h = bufs["h"][:st].float().cpu(), bufs["h"][st:].float().cpu()
    f_c, f_h = oflux.double_block(bw, hidden, context, temb, cos, sin, shape)
    if quant is None:
        e_c, e_h = rel_l2(out_c, f_c[0]), rel_l2(out_h, f_h[0])
        print(f"rel L2 vs fp32 oracle: context {e_c:.3e} hidden {e_h:.3e}", flush=True)
        parity("double block, text rows, rel L2 vs fp32 oracle", e_c, TOL[kind])
        parity("double block, image rows, rel L2 vs fp32 oracle", e_h, TOL[kind])
        assert e_c < TOL[kind] and e_h < TOL[kind]
        return
    mods = (_host_mods(dit, mod, ("d", 0, "norm1"), 6),
            _host_mods(dit, mod, ("d", 0, "norm1_context"), 6))
    ref_c, ref_h = oflux.double_block(bw, hidden, context, temb, cos, sin, shape, quant=quant,
                                      act_dtype=torch.bfloat16, store=torch.bfloat16, mods=mods)
    e_c, e_h = rel_l2(out_c, ref_c[0]), rel_l2(out_h, ref_h[0])
    q_c, q_h = rel_l2(out_c, f_c[0]), rel_l2(out_h, f_h[0])
    o_c, o_h = rel_l2(ref_c, f_c), rel_l2(ref_h, f_h)
    print(f"rel L2 vs same-law oracle: context {e_c:.3e} hidden {e_h:.3e}; {kind} format "
          f"error vs fp32: device {q_c:.3e} / {q_h:.3e}, oracle {o_c:.3e} / {o_h:.3e}", flush=True)
    parity(f"double block {kind}, text rows, rel L2 vs same-law oracle", e_c, TOL[kind])
    parity(f"double block {kind}, image rows, rel L2 vs same-law oracle", e_h, TOL[kind])
    parity(f"double block {kind}, image rows, format error vs fp32 (oracle's {o_h:.3e})", q_h,
           FORMAT_ERR)
    assert e_c < TOL[kind] and e_h < TOL[kind]
    assert abs(q_c - o_c) < 0.1 * o_c and abs(q_h - o_h) < 0.1 * o_h
    assert q_c < FORMAT_ERR and q_h < FORMAT_ERR


def _check_single(gpu, kind, quant, parity, st=None, img_hw=None):
    shape, w, dit, hidden, context, temb, st, img_hw = _block_setup(gpu, kind, st, img_hw)
    print(f"flux single block {kind}, {st} + {img_hw[0] * img_hw[1]} tokens", flush=True)
    cos, sin = ops.flux_pos_embed(ops.flux_ids(st, *img_hw))
    x = torch.cat([context, hidden], dim=1)
    bw = {k[len("single_transformer_blocks.0."):]: v for k, v in w.items()
          if k.startswith("single_transformer_blocks.0.")}
    bufs = dit._buffers(st, hidden.shape[1])
    bufs["h"].copy_(x[0].to(gpu, torch.bfloat16))
    mod = _gpu_mod(dit, temb, gpu)
    gcos, gsin = dit.rope_tables(st, img_hw)
    dit.single_block(0, bufs, mod, gcos, gsin)
    torch.cuda.synchronize()
    out = bufs["h"].float().cpu()
    full = oflux.single_block(bw, x, temb, cos, sin, shape)
    if quant is None:
        e = rel_l2(out, full[0])
        print(f"rel L2 vs fp32 oracle {e:.3e}", flush=True)
        parity("single block, rel L2 vs fp32 oracle", e, TOL[kind])
        assert e < TOL[kind]
        return
    ref = oflux.single_block(bw, x, temb, cos, sin, shape, quant=quant, act_dtype=torch.bfloat16,
                             store=torch.bfloat16, mods=_host_mods(dit, mod, ("s", 0), 3))
    e = rel_l2(out, ref[0])
    q, o = rel_l2(out, full[0]), rel_l2(ref, full)
    print(f"rel L2 vs same-law oracle {e:.3e}; {kind} format error vs fp32: device {q:.3e}, "
          f"oracle {o:.3e}", flush=True)
    parity(f"single block {kind}, rel L2 vs same-law oracle", e, TOL[kind])
    parity(f"single block {kind}, format error vs fp32 (oracle's {o:.3e})", q, FORMAT_ERR)
    assert e < TOL[kind]
    assert abs(q - o) < 0.1 * o
    assert q < FORMAT_ERR


@pytest.mark.parametrize("kind,quant", CASES)
def test_double_block_matches_fp32_oracle(gpu, kind, quant, parity):
    _check_double(gpu, kind, quant, parity)


@pytest.mark.parametrize("kind,quant", CASES)
def test_single_block_matches_fp32_oracle(gpu, kind, quant, parity):
    _check_single(gpu, kind, quant, parity)


# The FLUX.1-dev 1024^2 step's own block shape: 512 text + 64 x 64 image tokens (4608 rows),
# attention over 4608 keys on the split schedule, every GEMM at its step size.
@pytest.mark.parametrize("kind,quant", [("bf16", None), ("fp8", "fp8")])
def test_double_block_at_the_flux_1024_step_shape(gpu, kind, quant, parity):
    _check_double(gpu, kind, quant, parity, st=512, img_hw=(64, 64))


@pytest.mark.parametrize("kind,quant", [("bf16", None), ("fp8", "fp8")])
def test_single_block_at_the_flux_1024_step_shape(gpu, kind, quant, parity):
    _check_single(gpu, kind, quant, parity, st=512, img_hw=(64, 64))


def test_reduced_depth_step_matches_fp32_oracle(gpu, parity):
    """Embedders + 2 double + 2 single blocks + norm_out / proj_out at FLUX width, a 32 x 32
    patch grid and 256 text tokens: the whole step's wiring against the oracle's forward."""
    shape = oflux.FluxShape(n_double=2, n_single=2)
    cfg = FluxConfig(n_double=2, n_single=2)
    w = _source(shape, 2, 2)
    img_hw, st = (32, 32), 256
    inp = oflux.synthetic_inputs(shape, SEED, img_hw, st)
    inp = {k: (v.bfloat16().float() if k in ("latents", "text", "pooled") else v)
           for k, v in inp.items()}
    # a bf16 model casts timestep / guidance to bf16 and scales them there (:453-456,477-479)
    ref = oflux.forward(shape, SEED, inp["latents"], inp["text"], inp["pooled"],
                        inp["timestep"], inp["guidance"], img_hw, model_dtype=torch.bfloat16)
    dit = FluxDiT(cfg, lambda n: w[n], kind="bf16", device=gpu)
    out = dit.forward(inp["latents"].to(gpu), inp["text"].to(gpu), inp["pooled"].to(gpu),
                      inp["timestep"].to(gpu), inp["guidance"].to(gpu), img_hw)
    torch.cuda.synchronize()
    e = rel_l2(out, ref)
    print(f"step rel L2 {e:.3e}", flush=True)
    parity("2 + 2 block step, rel L2 vs fp32 oracle", e, 1e-2)
    assert out.shape == (1, 1024, 64)
    assert e < 1e-2
