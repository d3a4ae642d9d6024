"""The hot path at the configurations' own sizes on the GPU.

Attention at the step shapes against the fp32 oracle (every head of FLUX's 24 x 4608 x 4608 on
the split schedule; head and query subsets of Qwen's 7145-key, Wan's 32760-key self- and
512-key cross-attention, each subset checked over all keys). Wan's GEMMs at M = 32760 (bf16
q/k/v, FFN in and out with their epilogues, the MXFP8 FFN) over the first, last and scattered
tile rows against the oracle. The full-depth FLUX 1024^2 step (57 blocks, 4608 tokens) in bf16
and fp8 against the fp32 oracle's forward on the same weights. The Qwen-Image 1328^2 (60
blocks, MXFP8) and Wan 480p x 81 frames (40 blocks) steps through size-independent properties:
finite output and a bit-identical rerun. Block-level parity at these shapes is in
test_gpu_flux.py and test_gpu_qwen.py.
"""

import math

import pytest
import torch

from difflet_amd import kernels
from oracle import ops

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def _qkv(gpu, h, sq, sk, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    mk = lambda s: torch.randn(1, h, s, 128, generator=g, device=gpu).to(torch.bfloat16)  # noqa: E731
    return mk(sq), mk(sk), mk(sk)


def _check_rows(q, k, v, out, heads, rows, scale, tol=1e-2):
    """out[0, heads][:, rows] against fp32 CPU attention of those queries over every key."""
    idx = torch.as_tensor(rows, device=q.device)
    for hh in heads:
        qs = q[0, hh].index_select(0, idx).float().cpu()
        ref = ops.attention(qs[None], k[0, hh].float().cpu()[None], v[0, hh].float().cpu()[None],
                            scale=scale)[0]
        e = rel_l2(out[0, hh].index_select(0, idx), ref)
        assert e < tol, f"head {hh}: rel L2 {e:.3e}"


def test_flux_attention_24_heads_4608_split_schedule_every_head(gpu):
    """FLUX.1-dev 1024^2: 24 heads x (512 + 4096) tokens, the split schedule the step runs
    (432 query tiles of 256 on 256 CUs), every head and every query against fp32."""
    print("attention 1 x 24 x 4608 x 4608 (split schedule)", flush=True)
    q, k, v = _qkv(gpu, 24, 4608, 4608, 11)
    scale = 1 / math.sqrt(128)
    out = kernels.attention(q, k, v, scale=scale)
    again = kernels.attention(q, k, v, scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    _check_rows(q, k, v, out, range(24), range(4608), scale)


def test_qwen_attention_24_heads_7145(gpu):
    """Qwen-Image 1328^2: 24 heads x 7145 tokens (a ragged last query tile), six heads with
    the first, last and scattered query rows over all keys."""
    print("attention 1 x 24 x 7145 x 7145", flush=True)
    q, k, v = _qkv(gpu, 24, 7145, 7145, 12)
    scale = 1 / math.sqrt(128)
    out = kernels.attention(q, k, v, scale=scale)
    torch.cuda.synchronize()
    rows = list(range(256)) + list(range(7145 - 300, 7145)) + list(range(3000, 7145, 97))
    _check_rows(q, k, v, out, (0, 5, 11, 12, 17, 23), rows, scale)


def test_wan_self_attention_40_heads_32760_keys(gpu):
    """Wan 2.2 480p x 81 frames: 40 heads x 32760 tokens (5120 query tiles, 18 ms), four heads
    with the first tile, the ragged last tile and rows spread over the sequence."""
    print("attention 1 x 40 x 32760 x 32760", flush=True)
    q, k, v = _qkv(gpu, 40, 32760, 32760, 13)
    scale = 1 / math.sqrt(128)
    out = kernels.attention(q, k, v, scale=scale)
    torch.cuda.synchronize()
    rows = list(range(256)) + list(range(32760 - 248, 32760)) + list(range(300, 32760 - 248, 71))
    _check_rows(q, k, v, out, (0, 13, 26, 39), rows, scale)


def test_wan_cross_attention_40_heads_32760_queries_512_keys(gpu):
    """Wan's cross-attention: 32760 video queries over 512 text keys, every head on 2048
    query rows."""
    print("attention 1 x 40 x 32760 x 512", flush=True)
    q, k, v = _qkv(gpu, 40, 32760, 512, 14)
    scale = 1 / math.sqrt(128)
    out = kernels.attention(q, k, v, scale=scale)
    torch.cuda.synchronize()
    rows = list(range(0, 32760, 17))[:1900] + list(range(32760 - 148, 32760))
    _check_rows(q, k, v, out, range(40), rows, scale)


# ------------------------------------------------------------------------ full-depth steps
SEED = 20251


def _twice(step):
    a = step()
    b = step()
    torch.cuda.synchronize()
    return a, b


def _properties(name, a, b, shape):
    assert tuple(a.shape) == shape, f"{name}: shape {tuple(a.shape)}"
    assert torch.isfinite(a.float()).all(), f"{name}: non-finite output"
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{name}: rerun differs"
    assert a.float().std() > 0


# Full-depth FLUX bounds, from measured figures with a margin of about 1.45. bf16 against the
# fp32 oracle: 8.7e-3 over 2 + 2 blocks (test_gpu_flux.py), 1.37e-2 over the 57 (bf16 roundings
# of the residual stream and the modulation vectors, not a random walk: sqrt(57 / 4) would give
# 3.3e-2). fp8 against the same fp32 oracle is the e4m3 format's own error (per block 4.5-4.9e-2,
# equal to the same-law oracle's within 10 %, test_gpu_flux.py): 8.35e-2 over the 57 blocks.
FULL_BF16_TOL = 2e-2
FULL_FP8_TOL = 0.12


@pytest.mark.timeout(900)
def test_flux_full_depth_step_matches_the_oracle(gpu, parity, progress):
    """FLUX.1-dev 1024^2 (4096 + 512 tokens, 19 double + 38 single blocks) with random-init
    weights drawn on the device: bf16 and per-token fp8 steps, each finite and bit-identical
    on a rerun, against the oracle's fp32 forward over the same weights (fetched to the host one
    block at a time) and the same bf16-rounded inputs."""
    from difflet_amd.dit.flux import FluxConfig, FluxDiT, flux_param_shapes, random_param_source
    from oracle import flux as oflux

    torch.set_num_threads(16)
    cfg = FluxConfig()
    get = random_param_source(cfg, SEED, gpu)
    g = torch.Generator().manual_seed(SEED)
    lat = torch.randn(1, 4096, 64, generator=g).bfloat16().float()
    text = torch.randn(1, 512, 4096, generator=g).bfloat16().float()
    pooled = torch.randn(1, 768, generator=g).bfloat16().float()
    t = torch.rand(1, generator=g)
    guid = torch.full((1,), 3.5)
    outs = {}
    for kind in ("bf16", "fp8"):
        progress(f"flux full step {kind}")
        model = FluxDiT(cfg, get, kind=kind, device=gpu)
        a, b = _twice(lambda: model.forward(lat.to(gpu), text.to(gpu), pooled.to(gpu),
                                            t.to(gpu), guid.to(gpu), (64, 64)))
        _properties(f"flux {kind}", a, b, (1, 4096, 64))
        outs[kind] = a.float().cpu()
        del model, a, b
        torch.cuda.empty_cache()
    progress("flux full step: fp32 oracle forward, 57 blocks on the host")
    names = flux_param_shapes(cfg)
    host = lambda n: get(n).cpu().float()  # noqa: E731

    def blocks(prefix):
        keys = [n[len(prefix) + 3:] for n in names if n.startswith(prefix + ".0.")]

        def fetch(i):
            progress(f"  oracle {prefix} {i}")  # ~1.2 s of CPU per block
            return {k: host(f"{prefix}.{i}.{k}") for k in keys}

        return fetch

    ew = {n: host(n) for n in names if not n.startswith(("transformer_blocks.",
                                                        "single_transformer_blocks."))}
    ref = oflux.forward(oflux.FluxShape(), SEED, lat, text, pooled, t, guid, (64, 64),
                        weights=(ew, blocks("transformer_blocks"),
                                 blocks("single_transformer_blocks")),
                        model_dtype=torch.bfloat16)
    e_bf16, e_fp8 = rel_l2(outs["bf16"], ref), rel_l2(outs["fp8"], ref)
    e_pair = rel_l2(outs["fp8"], outs["bf16"])
    print(f"flux 57-block step rel L2 vs fp32 oracle: bf16 {e_bf16:.3e}, fp8 {e_fp8:.3e} "
          f"(fp8 vs bf16 {e_pair:.3e})", flush=True)
    parity("57-block FLUX 1024^2 step bf16, rel L2 vs fp32 oracle", e_bf16, FULL_BF16_TOL)
    parity("57-block FLUX 1024^2 step fp8, format error vs fp32 oracle", e_fp8, FULL_FP8_TOL)
    assert e_bf16 < FULL_BF16_TOL
    assert e_fp8 < FULL_FP8_TOL


# Wan's GEMMs at the step's M = 32760 (127 full 256-row tiles and a 248-row one): the first
# tile's rows, the last tile's and every 997th row between, against the oracle on the host.
WAN_M = 32760
WAN_ROWS = list(range(256)) + list(range(WAN_M - 248, WAN_M)) + list(range(300, WAN_M - 248, 997))


@pytest.mark.parametrize("name,n,k,kind,epi", [
    ("q/k/v", 15360, 5120, "bf16", "none"), ("ffn in", 13824, 5120, "bf16", "gelu"),
    ("ffn out", 5120, 13824, "bf16", "gate_residual"), ("ffn in", 13824, 5120, "mx", "gelu"),
    ("ffn out", 5120, 13824, "mx", "gate_residual")])
def test_wan_gemms_at_32760_rows(gpu, parity, name, n, k, kind, epi):
    from difflet_amd import _lib
    from difflet_amd.dit.linear import DeviceLinear, run
    from oracle import mx as omx

    print(f"wan gemm {name} {kind}: {WAN_M} x {n} x {k}", flush=True)
    torch.set_num_threads(16)
    g = torch.Generator(device=gpu).manual_seed(n + k)
    a = torch.randn(WAN_M, k, generator=g, device=gpu).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    b = (torch.randn(n, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    lin = DeviceLinear(w, b, kind)
    gate = res = None
    if epi == "gate_residual":
        gate = torch.randn(1, n, generator=g, device=gpu).to(torch.bfloat16)
        res = torch.randn(WAN_M, n, generator=g, device=gpu).to(torch.bfloat16)
        c = res.clone()
        run([lin.problem(a, c, gate=gate, residual=c)], kind, _lib.EPI_GATE_RESIDUAL)
    else:
        c = torch.empty(WAN_M, n, dtype=torch.bfloat16, device=gpu)
        run([lin.problem(a, c)], kind, _lib.EPI_GELU if epi == "gelu" else _lib.EPI_NONE)
    torch.cuda.synchronize()
    assert torch.isfinite(c.float()).all()
    idx = torch.as_tensor(WAN_ROWS, device=gpu)
    a_rows = a.index_select(0, idx).float().cpu()
    wf, bf = w.float().cpu(), b.float().cpu()
    if kind == "bf16":
        acc = ops.linear(a_rows, wf, bf)
    else:
        wq, ws = omx.quantize_mx(wf.numpy())
        acc = torch.from_numpy(omx.mx_linear(a_rows.numpy(), wq, ws, bf.numpy()))
    if epi == "gelu":
        ref = ops.gelu_tanh(acc)
    elif epi == "gate_residual":
        ref = res.index_select(0, idx).float().cpu() + gate.float().cpu() * acc
    else:
        ref = acc
    e = rel_l2(c.index_select(0, idx), ref)
    print(f"rel L2 over {len(WAN_ROWS)} rows {e:.3e}", flush=True)
    parity(f"Wan {name} GEMM {kind} {WAN_M} x {n} x {k}, rel L2 vs "
           f"{'fp32' if kind == 'bf16' else 'same-law'} oracle", e, 4e-3)
    assert e < 4e-3  # one bf16 rounding of the output


# Full-depth Qwen-Image bounds, from the measured figures with a margin of about 1.45 (as for FLUX
# above): bf16 against the fp32 oracle 2.05e-2 over the 60 blocks (5.6e-3 over 2, test_gpu_qwen.py:
# the bf16 roundings of the residual stream and the modulation vectors, again not a random walk,
# which would give 3.1e-2); MXFP8 against the same fp32 oracle is the format's own error (per
# block 4.6e-2, equal to the same-law oracle's, test_gpu_qwen.py), 1.00e-1 over the 60 blocks.
QWEN_FULL_BF16_TOL, QWEN_FULL_MX_TOL = 3e-2, 0.15


@pytest.mark.timeout(900)
def test_qwen_full_depth_step_matches_the_oracle(gpu, parity, progress):
    """Qwen-Image 1328^2 (6889 image + 256 text tokens, 60 joint blocks) with random-init weights
    drawn on the device: bf16 and MXFP8 steps, each finite and bit-identical on a rerun, against
    the oracle's fp32 forward over the same weights (fetched to the host one block at a time)
    and the same bf16-rounded inputs."""
    from difflet_amd.dit.qwen import QwenConfig, QwenImageDiT, qwen_param_shapes, random_param_source
    from oracle import qwen as oqwen

    torch.set_num_threads(16)
    cfg = QwenConfig()
    get = random_param_source(cfg, SEED, gpu)
    g = torch.Generator().manual_seed(SEED)
    lat = torch.randn(1, 6889, 64, generator=g).bfloat16().float()
    text = torch.randn(1, 256, 3584, generator=g).bfloat16().float()
    t = torch.rand(1, generator=g)
    outs = {}
    for kind in ("bf16", "mx"):
        progress(f"qwen full step {kind}")
        model = QwenImageDiT(cfg, get, kind=kind, device=gpu)
        a, b = _twice(lambda: model.forward(lat.to(gpu), text.to(gpu), t.to(gpu), (83, 83)))
        _properties(f"qwen {kind}", a, b, (1, 6889, 64))
        outs[kind] = a.float().cpu()
        del model, a, b
        torch.cuda.empty_cache()
    progress("qwen full step: fp32 oracle forward, 60 blocks on the host")
    names = qwen_param_shapes(cfg)
    host = lambda n: get(n).cpu().float()  # noqa: E731
    pre = "transformer_blocks."
    keys = [n[len(pre) + 2:] for n in names if n.startswith(pre + "0.")]

    class Blocks:
        def __getitem__(self, i):
            progress(f"  oracle block {i}")  # ~2 s of CPU per block
            return {k: host(f"{pre}{i}.{k}") for k in keys}

    ew = {n: host(n) for n in names if not n.startswith(pre)}
    ref = oqwen.forward(oqwen.QwenShape(), SEED, lat, text, t, (83, 83), weights=(ew, Blocks()),
                        model_dtype=torch.bfloat16)
    e_bf16, e_mx = rel_l2(outs["bf16"], ref), rel_l2(outs["mx"], ref)
    print(f"qwen 60-block step rel L2 vs fp32 oracle: bf16 {e_bf16:.3e}, mx {e_mx:.3e} "
          f"(mx vs bf16 {rel_l2(outs['mx'], outs['bf16']):.3e})", flush=True)
    parity("60-block Qwen-Image 1328^2 step bf16, rel L2 vs fp32 oracle", e_bf16, QWEN_FULL_BF16_TOL)
    parity("60-block Qwen-Image 1328^2 step MXFP8, format error vs fp32 oracle", e_mx,
           QWEN_FULL_MX_TOL)
    assert e_bf16 < QWEN_FULL_BF16_TOL
    assert e_mx < QWEN_FULL_MX_TOL


# Full-depth Wan bounds (40 blocks at width 5120 on a 5 x 24 x 26 latent: 780 video tokens, so
# the host oracle finishes in seconds; the GEMMs at the real 32760 rows are checked above), from
# the measured figures with a margin of about 1.45: bf16 against the fp32 oracle 1.33e-2 (4.9e-3
# over 2 blocks, test_gpu_wan.py), MXFP8 against the same oracle 3.29e-2, the format's error on
# the reference's Wan targets (a block's 1.5e-2, test_gpu_wan.py).
WAN_FULL_BF16_TOL, WAN_FULL_MX_TOL = 2e-2, 5e-2


@pytest.mark.timeout(900)
def test_wan_full_depth_step_matches_the_oracle(gpu, parity, progress):
    """Wan 2.2 14B's 40 blocks at full width (5120, 40 x 128 heads, FFN 13824) with random-init
    weights drawn on the device, on a 5 x 24 x 26 latent (780 video tokens) and 512 text tokens:
    bf16 and MXFP8 steps, each finite and bit-identical on a rerun, against the oracle's fp32
    forward over the same weights (fetched one block at a time) and the same bf16 inputs."""
    from difflet_amd.dit.wan import WanConfig, WanDiT, random_param_source, wan_param_shapes
    from oracle import wan as owan

    torch.set_num_threads(16)
    cfg = WanConfig()
    get = random_param_source(cfg, SEED, gpu)
    g = torch.Generator().manual_seed(SEED)
    lat = torch.randn(1, 16, 5, 24, 26, generator=g).bfloat16().float()
    text = torch.randn(1, 512, 4096, generator=g).bfloat16().float()
    t = torch.rand(1, generator=g) * 1000
    outs = {}
    for kind in ("bf16", "mx"):
        progress(f"wan full-depth step {kind}")
        model = WanDiT(cfg, get, device=gpu, kind=kind)
        a, b = _twice(lambda: model.forward(lat.to(gpu), t.to(gpu), text.to(gpu)))
        _properties(f"wan {kind}", a, b, (1, 16, 5, 24, 26))
        outs[kind] = a.float().cpu()
        del model, a, b
        torch.cuda.empty_cache()
    progress("wan full-depth step: fp32 oracle forward, 40 blocks on the host")
    names = wan_param_shapes(cfg)
    host = lambda n: get(n).cpu().float()  # noqa: E731
    pre = "blocks."
    keys = [n[len(pre) + 2:] for n in names if n.startswith(pre + "0.")]

    class Blocks:
        def __getitem__(self, i):
            progress(f"  oracle block {i}")
            return {k: host(f"{pre}{i}.{k}") for k in keys}

    ew = {n: host(n) for n in names if not n.startswith(pre)}
    ref = owan.forward(owan.WanShape(), SEED, lat, t, text, weights=(ew, Blocks()),
                       model_dtype=torch.bfloat16)
    e_bf16, e_mx = rel_l2(outs["bf16"], ref), rel_l2(outs["mx"], ref)
    progress(f"wan 40-block step rel L2 vs fp32 oracle: bf16 {e_bf16:.3e}, mx {e_mx:.3e} "
             f"(mx vs bf16 {rel_l2(outs['mx'], outs['bf16']):.3e})")
    parity("40-block Wan step (780 tokens) bf16, rel L2 vs fp32 oracle", e_bf16, WAN_FULL_BF16_TOL)
    parity("40-block Wan step (780 tokens) MXFP8, format error vs fp32 oracle", e_mx,
           WAN_FULL_MX_TOL)
    assert e_bf16 < WAN_FULL_BF16_TOL
    assert e_mx < WAN_FULL_MX_TOL


def test_qwen_full_step_60_blocks_mxfp8(gpu):
    """Qwen-Image 1328^2 (6889 + 256 tokens, 60 joint blocks) on the MXFP8 targets."""
    from difflet_amd.dit.qwen import QwenConfig, QwenImageDiT, random_param_source

    cfg = QwenConfig()
    g = torch.Generator(device=gpu).manual_seed(SEED)
    lat = torch.randn(1, 6889, 64, generator=g, device=gpu)
    text = torch.randn(1, 256, 3584, generator=g, device=gpu)
    t = torch.rand(1, generator=g, device=gpu)
    print("qwen full step mx", flush=True)
    model = QwenImageDiT(cfg, random_param_source(cfg, SEED, gpu), kind="mx", device=gpu)
    a, b = _twice(lambda: model.forward(lat, text, t, (83, 83)))
    _properties("qwen mx", a, b, (1, 6889, 64))
    del model
    torch.cuda.empty_cache()


def test_wan_full_step_40_blocks_bf16(gpu):
    """Wan 2.2 14B, 480 x 832 x 81 frames (latent 21 x 60 x 104, 32760 tokens) + 512 text
    tokens, 40 blocks, bf16."""
    from difflet_amd.dit.wan import WanConfig, WanDiT, random_param_source

    cfg = WanConfig()
    g = torch.Generator(device=gpu).manual_seed(SEED)
    lat = torch.randn(1, 16, 21, 60, 104, generator=g, device=gpu)
    text = torch.randn(1, 512, 4096, generator=g, device=gpu)
    t = torch.rand(1, generator=g, device=gpu) * 1000.0
    print("wan full step bf16", flush=True)
    model = WanDiT(cfg, random_param_source(cfg, SEED, gpu), device=gpu)
    a, b = _twice(lambda: model.forward(lat, t, text))
    _properties("wan bf16", a, b, (1, 16, 21, 60, 104))
    del model
    torch.cuda.empty_cache()
