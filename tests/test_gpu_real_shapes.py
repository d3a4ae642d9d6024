"""The hot path at the configurations' own sizes on the GPU.

Attention at the step shapes against the fp32 oracle (every head of FLUX's 24 x 4608 x 4608 on
the split schedule; head and query subsets of Qwen's 7145-key, Wan's 32760-key self- and
512-key cross-attention, each subset checked over all keys). The full-depth steps (FLUX
1024^2 57 blocks bf16 and fp8, Qwen-Image 1328^2 60 blocks MXFP8, Wan 480p x 81 frames 40
blocks bf16), whose CPU restatement would take hours, through size-independent properties:
finite output, a bit-identical rerun, and the fp8 step within a bound of the bf16 step.
Block-level parity at these shapes is in test_gpu_flux.py and test_gpu_qwen.py.
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


def test_flux_full_step_57_blocks_bf16_and_fp8(gpu):
    """FLUX.1-dev 1024^2 (4096 + 512 tokens, 19 double + 38 single blocks), random-init weights
    drawn on the device: both kinds finite and bit-identical on a rerun; the per-token fp8 step
    stays within 0.5 relative L2 of the bf16 step over the 57 blocks."""
    from difflet_amd.dit.flux import FluxConfig, FluxDiT, random_param_source

    cfg = FluxConfig()
    g = torch.Generator(device=gpu).manual_seed(SEED)
    lat = torch.randn(1, 4096, 64, generator=g, device=gpu)
    text = torch.randn(1, 512, 4096, generator=g, device=gpu)
    pooled = torch.randn(1, 768, generator=g, device=gpu)
    t = torch.rand(1, generator=g, device=gpu)
    guid = torch.full((1,), 3.5, device=gpu)
    outs = {}
    for kind in ("bf16", "fp8"):
        print(f"flux full step {kind}", flush=True)
        model = FluxDiT(cfg, random_param_source(cfg, SEED, gpu), kind=kind, device=gpu)
        a, b = _twice(lambda: model.forward(lat, text, pooled, t, guid, (64, 64)))
        _properties(f"flux {kind}", a, b, (1, 4096, 64))
        outs[kind] = a.float().cpu()
        del model, a, b
        torch.cuda.empty_cache()
    e = rel_l2(outs["fp8"], outs["bf16"])
    print(f"flux fp8 step vs bf16 step: rel L2 {e:.3e}", flush=True)
    assert e < 0.5


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
