"""Kernel-level parity of the HIP path against the oracle, through the C ABI.

Integer work (fp8 / E8M0 codes) must be bit-exact; floating-point results are compared by
relative L2 against fp32 CPU math on the same (already bf16-rounded) inputs, with the tolerance
written in each test.
"""

import math

import numpy as np
import pytest
import torch

from difflet_amd import _lib, kernels
from oracle import fp8 as ofp8
from oracle import mx as omx
from oracle import ops

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def rnd(g, *shape, std=1.0, dtype=torch.bfloat16):
    return (torch.randn(*shape, generator=g) * std).to(dtype)


# ------------------------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (300, 200, 128), (1, 64, 64),
                                   (513, 1028, 320), (4608, 3072, 3072)])
def test_gemm_bf16_matches_fp32(gpu, m, n, k):
    print(f"gemm_bf16 m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m * 7 + n)
    a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
    ref = ops.linear(a.float(), w.float(), b.float())
    out = kernels.linear(a.to(gpu), w.to(gpu), b.to(gpu))
    assert out.dtype == torch.bfloat16 and out.shape == (m, n)
    assert rel_l2(out, ref) < 4e-3  # one bf16 rounding of the output (2^-9 relative)


def test_gemm_bf16_no_bias_and_strided_views(gpu):
    g = torch.Generator().manual_seed(1)
    big = rnd(g, 320, 3 * 192)
    a = big[:, 192:384]  # row stride 576, K = 192
    w = rnd(g, 128, 192, std=0.05)
    ref = ops.linear(a.float(), w.float())
    c = torch.zeros(320, 2 * 128, dtype=torch.bfloat16, device=gpu)
    out = c[:, 128:]
    kernels.gemm_grouped([kernels.Problem(a.to(gpu), w.to(gpu), out)])
    assert rel_l2(out, ref) < 4e-3
    assert torch.count_nonzero(c[:, :128]) == 0  # nothing written outside the view


def test_gemm_epilogues_gelu_and_gate_residual(gpu):
    g = torch.Generator().manual_seed(2)
    m, n, k = 700, 512, 256
    a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
    pre = ops.linear(a.float(), w.float(), b.float())
    # GELU on columns >= 128 only
    out = kernels.linear(a.to(gpu), w.to(gpu), b.to(gpu), epilogue=_lib.EPI_GELU,
                         act_col_start=128)
    ref = torch.cat([pre[:, :128], ops.gelu_tanh(pre[:, 128:])], dim=1)
    assert rel_l2(out, ref) < 4e-3
    # residual + gate * (acc + bias), written in place over the residual
    gate, res = rnd(g, 1, n), rnd(g, m, n)
    ref2 = res.float() + gate.float() * pre
    r = res.to(gpu)
    kernels.gemm_grouped([kernels.Problem(a.to(gpu), w.to(gpu), r, b.to(gpu), gate.to(gpu), r)],
                         epilogue=_lib.EPI_GATE_RESIDUAL)
    assert rel_l2(r, ref2) < 4e-3


def _gemm_operands(kind, a, w, gpu):
    if kind == "bf16":
        return a.to(gpu), w.to(gpu), None, None
    if kind == "fp8":
        aq, sa = kernels.quantize_fp8_rowwise(a.to(gpu))
        wq, sw = kernels.quantize_fp8_rowwise(w.to(gpu))
        return aq, wq, sa, sw
    aq, sa = kernels.quantize_mxfp8(a.to(gpu), swizzled=True)
    wq, sw = kernels.quantize_mxfp8(w.to(gpu), swizzled=True)
    return aq, wq, sa, sw


def _rope_tables(g, rows):
    ang = torch.rand(rows, 64, generator=g) * 6.0
    cos = ang.cos().repeat_interleave(2, dim=1).contiguous()
    sin = ang.sin().repeat_interleave(2, dim=1).contiguous()
    sin[:, 0::2] *= 0.9  # distinct angles for the two elements of a pair (law 1 reads both)
    return cos, sin


@pytest.mark.parametrize("kind", ["bf16", "fp8", "mx"])
@pytest.mark.parametrize("law", [0, 1])
def test_gemm_fused_qk_norm_rope_equals_gemm_then_qk_norm_rope(gpu, kind, law):
    """Joint-block layout: text and image problems (ragged rows) write [q | k | v] of 4 heads;
    each problem has its own q/k norm weights and RoPE row offset. The fused epilogue equals
    the plain GEMM followed by qk_norm_rope within fp32 summation order."""
    print(f"fused qk gemm {kind} law={law}", flush=True)
    g = torch.Generator().manual_seed(40 + law)
    heads, d, k = 4, 512, 256
    mt, mi = 96, 300
    ws = [rnd(g, 3 * d, k, std=0.05) for _ in range(2)]
    bs = [rnd(g, 3 * d, std=0.1) for _ in range(2)]
    nw = [(1 + 0.3 * rnd(g, 128)).to(torch.bfloat16) for _ in range(4)]  # naq, nak, nq, nk
    a = rnd(g, mt + mi, k)
    cos, sin = (t.to(gpu) for t in _rope_tables(g, mt + mi))
    out = {}
    for fused in (True, False):
        buf = torch.full((mt + mi, 3 * d), float("nan"), dtype=torch.bfloat16, device=gpu)
        probs = []
        for p, rows in enumerate((slice(0, mt), slice(mt, mt + mi))):
            aq, wq, sa, sw = _gemm_operands(kind, a[rows], ws[p], gpu)
            probs.append(kernels.Problem(aq, wq, buf[rows], bs[p].to(gpu), a_scale=sa, w_scale=sw,
                                         norm_q=nw[2 * p].to(gpu), norm_k=nw[2 * p + 1].to(gpu),
                                         rope_row0=rows.start))
        qk = kernels.QkNormRope(0, d, d, cos, sin, law=law, eps=1e-6) if fused else None
        kernels.gemm_grouped(probs, kind=kind, qk=qk)
        if not fused:
            kernels.qk_norm_rope(buf, heads=heads, head_dim=128, q_off=0, k_off=d,
                                 wq=nw[0].to(gpu), wk=nw[1].to(gpu), eps=1e-6, cos=cos, sin=sin,
                                 law=law, split=mt, wq2=nw[2].to(gpu), wk2=nw[3].to(gpu))
        out[fused] = buf
    torch.cuda.synchronize()
    f, u = out[True], out[False]
    assert not torch.isnan(f).any()
    assert torch.equal(f[:, 2 * d:], u[:, 2 * d:])  # v untouched by the norm
    assert rel_l2(f, u) < 1e-3
    assert (f == u).float().mean().item() > 0.97  # most values bit-identical


def test_gemm_fused_qk_norm_rope_single_block_layout_and_errors(gpu):
    """[k | v | q | mlp] with GELU from the MLP columns: the norm on k and q, GELU on the MLP
    part, v plain; bad column ranges are refused before any launch."""
    g = torch.Generator().manual_seed(44)
    d, k, m = 256, 256, 333
    n = 3 * d + 4 * d
    a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
    nq, nk = (1 + 0.3 * rnd(g, 128)).to(torch.bfloat16), (1 + 0.3 * rnd(g, 128)).to(torch.bfloat16)
    cos, sin = (t.to(gpu) for t in _rope_tables(g, m))
    f = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    kernels.gemm_grouped([kernels.Problem(a.to(gpu), w.to(gpu), f, b.to(gpu), norm_q=nq.to(gpu),
                                          norm_k=nk.to(gpu))],
                         epilogue=_lib.EPI_GELU, act_col_start=3 * d,
                         qk=kernels.QkNormRope(2 * d, 0, d, cos, sin))
    u = kernels.linear(a.to(gpu), w.to(gpu), b.to(gpu), epilogue=_lib.EPI_GELU,
                       act_col_start=3 * d)
    kernels.qk_norm_rope(u, heads=2, head_dim=128, q_off=2 * d, k_off=0, wq=nq.to(gpu),
                         wk=nk.to(gpu), eps=1e-6, cos=cos, sin=sin, law=0)
    torch.cuda.synchronize()
    assert torch.equal(f[:, d:2 * d], u[:, d:2 * d]) and torch.equal(f[:, 3 * d:], u[:, 3 * d:])
    assert rel_l2(f, u) < 1e-3
    p = [kernels.Problem(a.to(gpu), w.to(gpu), f, b.to(gpu))]
    for bad, epi in ((kernels.QkNormRope(128, None, d, cos, sin), 0),      # not a multiple of 256
                     (kernels.QkNormRope(0, 256, 512, cos, sin), 0),        # overlapping ranges
                     (kernels.QkNormRope(2 * d, 0, d, cos, sin), _lib.EPI_GELU),  # GELU overlap
                     (kernels.QkNormRope(0, None, d, cos, sin), _lib.EPI_GATE_RESIDUAL)):
        with pytest.raises((ValueError, NotImplementedError)):
            kernels.gemm_grouped(p, epilogue=epi, act_col_start=d, qk=bad)


def test_gemm_grouped_problems_share_n_k(gpu):
    g = torch.Generator().manual_seed(3)
    n, k = 384, 192
    ms = [512, 37, 1000, 256]
    probs, refs = [], []
    for m in ms:
        a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
        c = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        probs.append(kernels.Problem(a.to(gpu), w.to(gpu), c, b.to(gpu)))
        refs.append(ops.linear(a.float(), w.float(), b.float()))
    kernels.gemm_grouped(probs)
    for p, r in zip(probs, refs):
        assert rel_l2(p.c, r) < 4e-3


def test_gemm_rejects_bad_shapes(gpu):
    a = torch.zeros(16, 100, dtype=torch.bfloat16, device=gpu)  # k not a multiple of 64
    w = torch.zeros(32, 100, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        kernels.linear(a, w)
    a = torch.zeros(16, 64, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(30, 64, dtype=torch.bfloat16, device=gpu)  # n not a multiple of 4
    with pytest.raises(ValueError):
        kernels.linear(a, w)


# ------------------------------------------------------------------------------ quantizers
# widths cover every register-resident path (one chunk of 2048 per thread up to 8) and the
# two-pass path beyond 16384 columns; fp32 rows always take the two-pass path
@pytest.mark.parametrize("rows,cols,dtype", [(7, 64, torch.bfloat16), (300, 3072, torch.bfloat16),
                                             (33, 15360, torch.bfloat16),
                                             (20, 12288, torch.float16),
                                             (9, 16384, torch.bfloat16),
                                             (5, 16400, torch.bfloat16),
                                             (6, 3000, torch.float32)])
def test_quantize_fp8_rowwise_bit_exact(gpu, rows, cols, dtype):
    print(f"quantize_fp8_rowwise rows={rows} cols={cols} {dtype}", flush=True)
    g = torch.Generator().manual_seed(rows + cols)
    x = (rnd(g, rows, cols) * torch.exp(torch.randn(rows, 1, generator=g) * 3).bfloat16()).to(dtype)
    x[0] = 0  # an all-zero row
    q, s = kernels.quantize_fp8_rowwise(x.to(gpu))
    q_ref, s_ref = ofp8.quantize_rowwise(x.float().numpy())
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_fp8_encode_every_code_and_rounding_midpoint(gpu):
    """The device encodes with the hardware conversion: every e4m3 value, every midpoint
    between neighbours (ties to even, including the subnormal ones and the one below the
    smallest subnormal), and values just off each midpoint, all in fp32 rows whose max is 448
    (scale 1, so these are the encoder's exact inputs), give the oracle's codes."""
    codes = np.arange(0, 0x7f, dtype=np.uint8)  # +0 .. 448 (0x7e); 0x7f is NaN
    vals = omx.e4m3_decode(codes).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    off = np.concatenate([np.nextafter(mids.astype(np.float32), np.float32(0)),
                          np.nextafter(mids.astype(np.float32), np.float32(1e9))])
    pos = np.concatenate([vals, mids, off, [2.0 ** -10, 2.0 ** -11, 1e-30, 1e-45]])
    row = np.concatenate([pos, -pos]).astype(np.float32)
    row = np.concatenate([[448.0], row]).astype(np.float32)
    row = np.pad(row, (0, (-row.size) % 8))
    x = torch.from_numpy(np.stack([row, row[::-1].copy()]))
    q, s = kernels.quantize_fp8_rowwise(x.to(gpu))
    q_ref, s_ref = ofp8.quantize_rowwise(x.numpy())
    assert np.array_equal(s.cpu().numpy(), np.ones(2, np.float32))
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    # the MX quantizer's encoder on the same values (one block scale per 32, E8M0 of 448 is 1)
    xm = x[:, :x.shape[1] // 128 * 128].contiguous()
    qm, sm = kernels.quantize_mxfp8(xm.to(gpu))
    qm_ref, sm_ref = omx.quantize_mx(xm.numpy())
    assert np.array_equal(sm.cpu().numpy(), sm_ref)
    assert np.array_equal(qm.view(torch.uint8).cpu().numpy(), qm_ref)


@pytest.mark.parametrize("rows,dim", [(5, 64), (512, 3072), (77, 5120)])
def test_layernorm_modulate_fp8_equals_layernorm_then_quantize(gpu, rows, dim):
    g = torch.Generator().manual_seed(rows * 3 + dim)
    x = rnd(g, rows, dim, std=2.0) + 0.5
    x[1] = 0.25  # a constant row: LN output is the shift alone
    sc, sh = rnd(g, 1, dim, std=0.3), rnd(g, 1, dim, std=0.3)
    q, s = kernels.layernorm_modulate_fp8(x.to(gpu), sc.to(gpu), sh.to(gpu), eps=1e-6)
    y = kernels.layernorm_modulate(x.to(gpu), sc.to(gpu), sh.to(gpu), eps=1e-6)
    q2, s2 = kernels.quantize_fp8_rowwise(y)
    assert q.dtype == q2.dtype == torch.float8_e4m3fn
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)
    # and the per-row law of the oracle applied to the bf16 LayerNorm output
    q_ref, s_ref = ofp8.quantize_rowwise(y.float().cpu().numpy())
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    # the bf16 LayerNorm output itself against the fp32 closed form
    ref = ops.ada_modulate(x.float()[None], sh.float(), sc.float())[0]
    assert rel_l2(y, ref) < 4e-3


@pytest.mark.parametrize("rows,cols,gelu_from", [(37, 15360, 3072), (300, 12288, 0),
                                                  (5, 640, 8), (9, 16384, 16376)])
def test_quantize_fp8_rowwise_gelu_equals_gelu_then_quantize(gpu, rows, cols, gelu_from):
    """The per-token fp8 quantizer that applies the MLP's GELU from gelu_from on: codes and
    scales equal the GELU kernel's bf16 output (the values a GELU epilogue stores) quantized by
    the plain row quantizer, bit for bit."""
    g = torch.Generator().manual_seed(rows + cols)
    x = (rnd(g, rows, cols, std=2.0).float() * torch.exp(torch.randn(rows, 1, generator=g))).bfloat16()
    x[1, gelu_from:] = -30.0  # GELU of large negatives: zeros (and -0.0)
    xd = x.to(gpu)
    q, s = kernels.quantize_fp8_rowwise(xd, gelu_from=gelu_from)
    y = xd.clone()
    y[:, gelu_from:] = kernels.gelu_tanh(xd[:, gelu_from:])
    q2, s2 = kernels.quantize_fp8_rowwise(y)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)
    # strided input (W2's A operand is a column window of the single block's buffer)
    wide = torch.zeros(rows, cols + 64, dtype=torch.bfloat16, device=gpu)
    wide[:, 64:] = xd
    q3, s3 = kernels.quantize_fp8_rowwise(wide[:, 64:], gelu_from=gelu_from)
    torch.cuda.synchronize()
    assert torch.equal(q3.view(torch.uint8), q.view(torch.uint8)) and torch.equal(s3, s)


# (rows, dim, split, mod dtype, one_plus): a joint launch (text rows below `split` with their own
# vectors) at FLUX / Qwen width, Wan's fp32 vectors and its affine norm2 (one_plus off), and
# the narrowest / widest dims (one and sixteen swizzle tiles)
@pytest.mark.parametrize("rows,dim,split,mdt,one_plus", [
    (700, 3072, 100, torch.bfloat16, True), (333, 5120, 0, torch.float32, True),
    (129, 5120, 0, torch.bfloat16, False), (64, 512, 0, torch.bfloat16, True),
    (40, 8192, 7, torch.float32, True)])
def test_layernorm_modulate_mx_equals_layernorm_then_quantize(gpu, rows, dim, split, mdt,
                                                              one_plus):
    """The fused LayerNorm -> MXFP8 kernel against the bf16 LayerNorm followed by the swizzled
    MX quantizer (codes and E8M0 scales bit for bit) and the oracle's MX law on the same bf16
    rows."""
    print(f"layernorm_modulate_mx rows={rows} dim={dim} split={split} {mdt}", flush=True)
    g = torch.Generator().manual_seed(rows + dim)
    x = (rnd(g, rows, dim, std=2.0).float() * torch.exp(torch.randn(rows, 1, generator=g) * 3)
         + 0.5).bfloat16()
    x[1] = 0.25  # a constant row: LN output is the shift alone
    mods = (torch.randn(4, dim, generator=g) * 0.3).to(mdt).to(gpu)
    mods[2, :dim // 2] = 0  # a zero half: blocks of shift alone
    kw = dict(eps=1e-6, one_plus=one_plus)
    if split:
        kw.update(split=split, mul2=mods[2], add2=mods[3])
    xd = x.to(gpu)
    q, s = kernels.layernorm_modulate_mx(xd, mods[0], mods[1], **kw)
    y = kernels.layernorm_modulate(xd, mods[0], mods[1], **kw)
    q2, s2 = kernels.quantize_mxfp8(y, swizzled=True)
    torch.cuda.synchronize()
    assert q.dtype == torch.float8_e4m3fn and s.shape == (rows, dim // 32)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)
    q_ref, s_ref = omx.quantize_mx(y.float().cpu().numpy(), swizzled_out=True)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    # into strided outputs (the step's buffers are views of wider rows)
    qb = torch.zeros(rows, dim + 512, dtype=torch.uint8, device=gpu)
    sb = torch.zeros(rows, dim // 32 + 16, dtype=torch.uint8, device=gpu)
    kernels.layernorm_modulate_mx(xd, mods[0], mods[1], out=(qb[:, :dim].view(torch.float8_e4m3fn),
                                                             sb[:, :dim // 32]), **kw)
    torch.cuda.synchronize()
    assert torch.equal(qb[:, :dim], q.view(torch.uint8)) and torch.equal(sb[:, :dim // 32], s)
    assert int(qb[:, dim:].count_nonzero()) == 0 and int(sb[:, dim // 32:].count_nonzero()) == 0


def test_layernorm_modulate_mx_refuses_partial_tiles(gpu):
    x = torch.zeros(4, 640, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        kernels.layernorm_modulate_mx(x, None, None, eps=1e-6)


@pytest.mark.parametrize("cols", [128, 384, 512, 896, 3072, 3456, 13824])
@pytest.mark.parametrize("swizzled", [False, True])
def test_quantize_mxfp8_bit_exact(gpu, cols, swizzled):
    g = torch.Generator().manual_seed(cols)
    rows = 19
    x = rnd(g, rows, cols) * torch.exp(torch.randn(rows, cols, generator=g) * 2).bfloat16()
    x[1, :] = 0
    x[2, 5] = 1e4  # an outlier in one block
    x[3, :32] = 1e-30  # tiny block (scale clamps at 0)
    q, s = kernels.quantize_mxfp8(x.to(gpu), swizzled=swizzled)
    q_ref, s_ref = omx.quantize_mx(x.float().numpy(), swizzled_out=swizzled)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


@pytest.mark.parametrize("kind", ["bf16", "mx"])
def test_gemm_gate_residual_short_problems_read_only_their_gate_row(gpu, kind):
    """Problems of 64 and 255 rows (one batch each) whose gate is one row of a much wider
    modulation buffer: every wave, including those whose rows lie past M, reads that row only."""
    print(f"gemm gate/residual short problems {kind}", flush=True)
    g = torch.Generator().manual_seed(77)
    n, k = 512, 256
    wide = rnd(g, 1, 40 * n, std=0.5)  # like the stacked adaLN vectors: gate = a [1, n] slice
    w, b = rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
    gate = wide.to(gpu)[:, 3 * n:4 * n]
    probs, refs = [], []
    for m in (64, 255):
        a, res = rnd(g, m, k), rnd(g, m, n)
        c = res.to(gpu).clone()
        if kind == "mx":
            aq, asc = kernels.quantize_mxfp8(a.to(gpu), swizzled=True)
            wq, ws = kernels.quantize_mxfp8(w.to(gpu), swizzled=True)
            wq_l, ws_l = omx.quantize_mx(w.float().numpy())
            y = torch.from_numpy(omx.mx_linear(a.float().numpy(), wq_l, ws_l, b.float().numpy()))
            probs.append(kernels.Problem(aq, wq, c, b.to(gpu), gate, c, a_scale=asc, w_scale=ws))
        else:
            y = a.float() @ w.float().T + b.float()
            probs.append(kernels.Problem(a.to(gpu), w.to(gpu), c, b.to(gpu), gate, c))
        refs.append((c, res.float() + gate.float().cpu() * y))
    kernels.gemm_grouped(probs, kind=kind, epilogue=_lib.EPI_GATE_RESIDUAL)
    torch.cuda.synchronize()
    for c, ref in refs:
        assert rel_l2(c, ref) < 4e-3


@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (300, 520, 384), (4608, 3072, 3072)])
def test_gemm_fp8_rowwise_matches_oracle(gpu, m, n, k):
    print(f"gemm_fp8 m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
    wq, ws = kernels.quantize_fp8_rowwise(w.to(gpu))
    aq, as_ = kernels.quantize_fp8_rowwise(a.to(gpu))
    c = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    kernels.gemm_grouped([kernels.Problem(aq, wq, c, b.to(gpu), a_scale=as_, w_scale=ws)],
                         kind="fp8")
    wq_ref, ws_ref = ofp8.quantize_rowwise(w.float().numpy())
    ref = ofp8.fp8_linear(a.float().numpy(), wq_ref, ws_ref, b.float().numpy())
    assert rel_l2(c, torch.from_numpy(ref)) < 4e-3  # same codes; fp32 sum order + bf16 out


# K of 1 to 24 stages of 128: scale blocks of four stages, the last one partial at k = 384,
# 640 and 1152 (the scale ring's 16-byte rows then end inside the next row's bytes)
@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (300, 520, 384), (200, 384, 640),
                                   (513, 260, 1152), (1030, 1024, 3072)])
def test_gemm_mxfp8_matches_fake_quant_linear(gpu, m, n, k):
    print(f"gemm_mx m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m * 3 + k)
    a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
    a[0, 7] = 50.0  # an outlier block
    a[1, k - 5] = -30.0  # in the last block of row 1
    w[3, k // 2 + 1] = 2.0  # a weight block with its own scale
    wq, ws = kernels.quantize_mxfp8(w.to(gpu), swizzled=True)
    aq, as_ = kernels.quantize_mxfp8(a.to(gpu), swizzled=True)
    c = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    kernels.gemm_grouped([kernels.Problem(aq, wq, c, b.to(gpu), a_scale=as_, w_scale=ws)],
                         kind="mx")
    wq_l, ws_l = omx.quantize_mx(w.float().numpy())
    ref = omx.mx_linear(a.float().numpy(), wq_l, ws_l, b.float().numpy())
    assert rel_l2(c, torch.from_numpy(ref)) < 4e-3


# (m, n, k, split rows, workspace): a two-problem launch (text / image rows), FLUX-Qwen's MLP
# width, a width with a 128-wide last swizzle tile, and 336 tiles on the split schedule
@pytest.mark.parametrize("m,n,k,split,ws", [(300, 1024, 512, 0, None), (900, 12288, 3072, 256, None),
                                            (500, 640, 256, 77, None),
                                            (7168, 3072, 3072, 0, "shared")])
def test_gemm_gelu_mx_epilogue_equals_gelu_then_quantize(gpu, m, n, k, split, ws):
    """The GELU -> MXFP8 epilogue of an MXFP8 GEMM whose weight rows are in swizzle order: its
    codes and E8M0 scales equal the swizzled MX quantizer applied to the bf16 GELU output of the
    same GEMM on the weights in logical order, bit for bit (the next GEMM's A operand)."""
    from difflet_amd.dit.linear import DeviceLinear

    print(f"gemm_mx gelu->mx m={m} n={n} k={k} split={split} ws={ws}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
    w[5] *= 40  # one output column with large values (its blocks scale alone)
    lin = DeviceLinear(w.to(gpu), b.to(gpu), "mx")
    aq, as_ = kernels.quantize_mxfp8(a.to(gpu), swizzled=True)
    rows = [slice(0, split), slice(split, m)] if split else [slice(0, m)]
    c = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    kernels.gemm_grouped([lin.problem(None, c[r], prepared=(aq[r], as_[r])) for r in rows],
                         kind="mx", epilogue=_lib.EPI_GELU, workspace=ws)
    q_ref, s_ref = kernels.quantize_mxfp8(c, swizzled=True)
    perm = lin.rows_in_swizzle_order()
    q = torch.full((m, n), 0x7f, dtype=torch.uint8, device=gpu).view(torch.float8_e4m3fn)
    s = torch.full((m, n // 32), 0xee, dtype=torch.uint8, device=gpu)
    kernels.gemm_grouped([perm.problem(None, q[r], prepared=(aq[r], as_[r]), c_scale=s[r])
                          for r in rows], kind="mx", epilogue=_lib.EPI_GELU_MX, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref)
    assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8))


def test_gemm_gelu_mx_epilogue_refusals(gpu):
    a = torch.zeros(64, 256, dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(96, 256, dtype=torch.bfloat16, device=gpu)
    q = torch.zeros(64, 96, dtype=torch.uint8, device=gpu)
    s = torch.zeros(64, 3, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError):  # bf16 GEMM
        kernels.gemm_grouped([kernels.Problem(a, w, q, c_scale=s)], kind="bf16",
                             epilogue=_lib.EPI_GELU_MX)
    aq, as_ = kernels.quantize_mxfp8(a, swizzled=True)
    wq, ws = kernels.quantize_mxfp8(w, swizzled=True)
    with pytest.raises(ValueError):  # no scale output
        kernels.gemm_grouped([kernels.Problem(aq, wq, q, a_scale=as_, w_scale=ws)], kind="mx",
                             epilogue=_lib.EPI_GELU_MX)
    w2, = kernels.quantize_mxfp8(torch.zeros(80, 256, dtype=torch.bfloat16, device=gpu),
                                 swizzled=True)[:1]
    with pytest.raises(ValueError):  # n % 32 != 0
        kernels.gemm_grouped([kernels.Problem(aq, w2, q[:, :80], a_scale=as_,
                                              w_scale=torch.zeros(80, 8, dtype=torch.uint8,
                                                                  device=gpu),
                                              c_scale=s)], kind="mx", epilogue=_lib.EPI_GELU_MX)


# ------------------------------------------------------------------------------- attention
def _attn_case(g, b, h, sq, sk, d=128, dtype=torch.bfloat16):
    q, k, v = rnd(g, b, h, sq, d, dtype=dtype), rnd(g, b, h, sk, d, dtype=dtype), rnd(g, b, h, sk, d, dtype=dtype)
    return q, k, v


# seq_k > 1024 runs the ping-pong kernel (256 queries per workgroup): ragged query and key
# counts, a single query, 17 / 18 / 32 key tiles, several batches and heads
@pytest.mark.parametrize("b,h,sq,sk", [(1, 2, 128, 64), (1, 3, 200, 333), (2, 2, 77, 1000),
                                       (1, 2, 4608, 4608), (1, 2, 3000, 512), (1, 2, 300, 1025),
                                       (2, 3, 777, 1100), (1, 1, 1, 2048), (1, 2, 513, 1088)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_matches_fp32(gpu, b, h, sq, sk, dtype):
    print(f"attention b={b} h={h} sq={sq} sk={sk} {dtype}", flush=True)
    g = torch.Generator().manual_seed(sq + sk)
    q, k, v = _attn_case(g, b, h, sq, sk, dtype=dtype)
    scale = 1 / math.sqrt(128)
    ref = ops.attention(q.float(), k.float(), v.float(), scale=scale)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=scale)
    assert out.dtype == dtype and out.shape == q.shape
    assert rel_l2(out, ref) < 1e-2  # probabilities rounded to 16 bits before P V


# more 256-query tiles than compute units with a last wave under 90 % full: the split schedule
# (a round of whole tiles, then the rest cut along the keys over lockstep sets of workgroups and
# merged by the last contributor) runs with the workspace. On 256 CUs: 432 tiles of 18 key
# tiles cut 176 in sets of 16; 320 of 32 cut 64 in sets of 32; 300 of 18 cut 44 in sets of 16,
# the last group holding 12 tiles.
@pytest.mark.parametrize("b,h,sq,sk", [(1, 24, 4600, 1100), (2, 20, 2048, 2048),
                                       (1, 25, 3000, 1100)])
def test_attention_split_schedule_equals_whole_tiles(gpu, b, h, sq, sk):
    print(f"attention split b={b} h={h} sq={sq} sk={sk}", flush=True)
    g = torch.Generator().manual_seed(sq + sk + h)
    q, k, v = (t.to(gpu) for t in _attn_case(g, b, h, sq, sk))
    scale = 1 / math.sqrt(128)
    ws = kernels.attention_workspace(torch.device(gpu))
    split1 = kernels.attention(q, k, v, scale=scale, workspace=ws)
    split2 = kernels.attention(q, k, v, scale=scale, workspace=ws)
    whole = kernels.attention(q, k, v, scale=scale, workspace=None)
    torch.cuda.synchronize()
    assert torch.equal(split1.view(torch.int16), split2.view(torch.int16))  # deterministic
    assert not torch.isnan(split1).any()
    # merged parts sum in another order than one pass: a bf16 rounding step apart at most
    assert rel_l2(split1, whole) < 2e-3
    assert int(torch.count_nonzero(ws[:16384].view(torch.int32))) == 0  # counters back at zero
    ref = ops.attention(q[:1, :2].float().cpu(), k[:1, :2].float().cpu(), v[:1, :2].float().cpu(),
                        scale=scale)
    assert rel_l2(split1[:1, :2], ref) < 1e-2


def test_attention_split_schedule_on_two_streams(gpu):
    """The shared split-schedule workspace is per stream: attention launched on two streams at
    once uses two workspaces, and both results equal the unsplit ones."""
    g = torch.Generator().manual_seed(77)
    dev = torch.device(gpu)
    cases = [tuple(t.to(gpu) for t in _attn_case(g, 1, 24, 4600, 1100)) for _ in range(2)]
    scale = 1 / math.sqrt(128)
    wholes = [kernels.attention(*c, scale=scale, workspace=None) for c in cases]
    streams = [torch.cuda.Stream(device=dev) for _ in range(2)]
    torch.cuda.synchronize()
    outs = []
    for c, st in zip(cases, streams):
        with torch.cuda.stream(st):
            outs.append(kernels.attention(*c, scale=scale))
    torch.cuda.synchronize()
    wss = []
    for st in streams:
        with torch.cuda.stream(st):
            wss.append(kernels.attention_workspace(dev))
    assert wss[0].data_ptr() != wss[1].data_ptr()
    for o, w in zip(outs, wholes):
        assert rel_l2(o, w) < 2e-3


@pytest.mark.parametrize("ramp", [False, True])
def test_attention_large_and_growing_scores(gpu, ramp):
    """Scores far outside exp2's range (softmax scale folded: |s| up to ~60 in log2 units) and,
    with the ramp, keys whose magnitude grows along the sequence, so the running max jumps by
    more than 20 on later tiles: the ping-pong kernel's rescaling path against fp32."""
    g = torch.Generator().manual_seed(31 + ramp)
    b, h, sq, sk = 1, 2, 600, 2000
    q, k, v = _attn_case(g, b, h, sq, sk)
    q = (q.float() * 3).to(torch.bfloat16)
    k = k.float() * 3
    if ramp:
        k = k * torch.linspace(0.2, 3.0, sk).view(1, 1, sk, 1)
    k = k.to(torch.bfloat16)
    scale = 1 / math.sqrt(128)
    ref = ops.attention(q.float(), k.float(), v.float(), scale=scale)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=scale)
    assert torch.isfinite(out.float()).all()
    assert rel_l2(out, ref) < 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("jump", [15.5, 17.0, 19.5])
def test_attention_late_key_beats_the_running_max(gpu, dtype, jump):
    """One key on a late tile scores `jump` log2 units above every earlier key (scale 1: a
    score of jump / log2(e)). Unrescaled its probability would be 2^jump, past fp16's 65504
    from 2^16 on: the ping-pong kernel must rescale before packing P for fp16 as for bf16."""
    g = torch.Generator().manual_seed(int(jump * 10))
    b, h, sq, sk, hot = 1, 2, 300, 2000, 1500
    q = torch.randn(b, h, sq, 128, generator=g) * 0.02
    k = torch.randn(b, h, sk, 128, generator=g) * 0.02
    v = torch.randn(b, h, sk, 128, generator=g)
    q[..., 0] = 1.0
    k[..., 0] = 0.0
    k[:, :, hot, 0] = jump / math.log2(math.e)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    ref = ops.attention(q.float(), k.float(), v.float(), scale=1.0)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=1.0)
    assert torch.isfinite(out.float()).all()
    err = rel_l2(out, ref)
    print(f"attention late jump {jump} {dtype}: rel L2 {err:.2e}", flush=True)
    assert err < 1e-2


def test_attention_folded_heads_and_scale_one(gpu):
    g = torch.Generator().manual_seed(5)
    q, k, v = (rnd(g, 6, 96, 128, std=0.2) for _ in range(3))
    ref = ops.attention(q.float(), k.float(), v.float(), scale=None)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=1.0)
    assert out.shape == (6, 96, 128)
    assert rel_l2(out, ref) < 1e-2


def test_attention_causal_bool_and_additive_masks(gpu):
    g = torch.Generator().manual_seed(6)
    q, k, v = _attn_case(g, 1, 2, 150, 150)
    s = 0.1
    qf, kf, vf = q.float(), k.float(), v.float()
    ref = ops.attention(qf, kf, vf, scale=s, causal=True)
    assert rel_l2(kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=s, causal=True), ref) < 1e-2
    mask = torch.rand(150, 150, generator=g) > 0.3
    ref = ops.attention(qf, kf, vf, scale=s, attention_mask=mask)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=s, attention_mask=mask.to(gpu))
    assert rel_l2(out, ref) < 1e-2
    add = torch.randn(1, 2, 150, 150, generator=g)
    ref = ops.attention(qf, kf, vf, scale=s, attention_mask=add)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=s, attention_mask=add.to(gpu))
    assert rel_l2(out, ref) < 1e-2


def test_attention_bounds_equal_mask_and_fully_masked_rows_average_v(gpu):
    """tests/unit/backends/test_cpu_ops_impl.py:492-517: bounds are the contiguous key window;
    a row with no valid key averages v (softmax over equal finfo.min scores)."""
    g = torch.Generator().manual_seed(7)
    bh, s = 4, 300
    q, k, v = (rnd(g, bh, s, 128) for _ in range(3))
    bmin = torch.randint(0, 100, (bh, s, 1), generator=g, dtype=torch.int32)
    bmax = bmin + torch.randint(1, 200, (bh, s, 1), generator=g, dtype=torch.int32)
    bmax[0, :10] = bmin[0, :10]  # empty window
    ref = ops.attention(q.float(), k.float(), v.float(), scale=0.05, bound_min=bmin,
                        bound_max=bmax)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=0.05,
                            bound_min=bmin.to(gpu), bound_max=bmax.to(gpu))
    assert rel_l2(out, ref) < 1e-2
    mean_v = v[0].float().mean(dim=0)
    assert rel_l2(out[0, :10].float().cpu(), mean_v.expand(10, -1)) < 1e-2
    with pytest.raises(ValueError):
        kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=1.0, bound_min=bmin.to(gpu))


@pytest.mark.parametrize("s", [333, 1500])
def test_attention_strided_inplace_over_q(gpu, s):
    """The DiT layout: q/k/v are column ranges of one [S, 3D] buffer; output over q."""
    g = torch.Generator().manual_seed(8)
    hds = 3
    d = hds * 128
    buf = rnd(g, s, 3 * d)
    ref_q, ref_k, ref_v = (buf[:, i * d:(i + 1) * d].reshape(s, hds, 128).transpose(0, 1).float()
                           for i in range(3))
    ref = ops.attention(ref_q, ref_k, ref_v, scale=0.08).transpose(0, 1).reshape(s, d)
    gb = buf.to(gpu)
    view = lambda off: gb.as_strided((1, hds, s, 128), (0, 128, 3 * d, 1), off)  # noqa: E731
    q = view(0)
    kernels.attention(q, view(d), view(2 * d), scale=0.08, out=q)
    assert rel_l2(gb[:, :d], ref) < 1e-2
    assert torch.equal(gb[:, d:].cpu(), buf[:, d:])  # k, v untouched


# --------------------------------------------------------------------- norms, rope, misc
@pytest.mark.parametrize("rows,dim", [(5, 64), (4608, 3072), (130, 5120)])
def test_layernorm_modulate(gpu, rows, dim):
    g = torch.Generator().manual_seed(rows)
    x = rnd(g, rows, dim, std=2.0) + 0.5
    sc, sh = rnd(g, 1, dim, std=0.3), rnd(g, 1, dim, std=0.3)
    ref = ops.ada_modulate(x.float()[None], sh.float(), sc.float())[0]
    out = kernels.layernorm_modulate(x.to(gpu), sc.to(gpu), sh.to(gpu), eps=1e-6)
    assert rel_l2(out, ref) < 4e-3
    # plain affine LayerNorm and fp32 in / bf16 out
    w, b = rnd(g, dim, dtype=torch.float32), rnd(g, dim, dtype=torch.float32)
    ref = torch.nn.functional.layer_norm(x.float(), (dim,), w, b, eps=1e-5)
    out = kernels.layernorm_modulate(x.float().to(gpu), w.to(gpu), b.to(gpu), eps=1e-5,
                                     one_plus=False, out_dtype=torch.bfloat16)
    assert out.dtype == torch.bfloat16 and rel_l2(out, ref) < 4e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rms_norm_fp32_law(gpu, dtype):
    g = torch.Generator().manual_seed(9)
    x = rnd(g, 37, 5120, dtype=dtype)
    w = (torch.rand(5120, generator=g) + 0.5).to(dtype)
    ref = ops.rms_norm_fp32(x, w, 1e-6)
    out = kernels.rms_norm(x.to(gpu), w.to(gpu), 1e-6)
    tol = 1e-6 if dtype == torch.float32 else 4e-3
    assert rel_l2(out, ref) < tol


def test_qk_norm_rope_in_place(gpu):
    g = torch.Generator().manual_seed(10)
    s, h = 520, 24
    d = h * 128
    buf = rnd(g, s, 3 * d)
    wq = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    wk = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    ids = ops.flux_ids(8, 16, 32)
    cos, sin = ops.flux_pos_embed(ids)
    def ref_of(off, w):
        x = buf[:, off:off + d].float().reshape(s, h, 128).transpose(0, 1)
        x = ops.rms_norm_fp32(x, w.float(), 1e-6)
        return ops.apply_rotary_emb_fp32(x, cos[None], sin[None]).transpose(0, 1).reshape(s, d)
    rq, rk = ref_of(0, wq), ref_of(d, wk)
    gb = buf.to(gpu)
    kernels.qk_norm_rope(gb, heads=h, head_dim=128, q_off=0, k_off=d, wq=wq.to(gpu),
                         wk=wk.to(gpu), eps=1e-6, cos=cos.to(gpu), sin=sin.to(gpu), law=0)
    assert rel_l2(gb[:, :d], rq) < 4e-3
    assert rel_l2(gb[:, d:2 * d], rk) < 4e-3
    assert torch.equal(gb[:, 2 * d:].cpu(), buf[:, 2 * d:])


@pytest.mark.parametrize("h,wdt,law", [(40, torch.float32, 1), (40, torch.bfloat16, 0),
                                       (16, torch.float32, 1), (5, torch.float32, 1)])
def test_qk_norm_across_heads_in_place(gpu, h, wdt, law):
    """do_norm 2 (Wan): one RMS over all heads of q (and of k) with [heads * 128] weights, then
    RoPE per head; 16 / 40 heads hold whole rows in registers, 5 heads take the general kernel.
    A q-only call leaves k untouched."""
    print(f"qk across heads h={h} {wdt} law={law}", flush=True)
    g = torch.Generator().manual_seed(h + law)
    s, d = 300, h * 128
    buf = rnd(g, s, 3 * d)
    wq = (1 + 0.1 * torch.randn(d, generator=g)).to(wdt)
    wk = (1 + 0.1 * torch.randn(d, generator=g)).to(wdt)
    ang = torch.rand(s, 64, generator=g) * 6.0
    cos = ang.cos().repeat_interleave(2, dim=1).contiguous()
    sin = ang.sin().repeat_interleave(2, dim=1).contiguous()
    rot = ops.apply_rotary_emb_fp32 if law == 0 else ops.apply_rotary_emb
    def ref_of(off, w):
        x = ops.rms_norm_fp32(buf[:, off:off + d].float(), w.float(), 1e-6).reshape(s, h, 128)
        return rot(x, cos[:, None], sin[:, None]).reshape(s, d)
    gb = buf.to(gpu)
    kernels.qk_norm_rope(gb, heads=h, head_dim=128, q_off=0, k_off=d, wq=wq.to(gpu),
                         wk=wk.to(gpu), eps=1e-6, cos=cos.to(gpu), sin=sin.to(gpu), law=law,
                         do_norm=2)
    assert rel_l2(gb[:, :d], ref_of(0, wq)) < 4e-3
    assert rel_l2(gb[:, d:2 * d], ref_of(d, wk)) < 4e-3
    assert torch.equal(gb[:, 2 * d:].cpu(), buf[:, 2 * d:])
    gq = buf.to(gpu)
    kernels.qk_norm_rope(gq, heads=h, head_dim=128, q_off=0, k_off=-1, wq=wq.to(gpu), wk=None,
                         eps=1e-6, cos=cos.to(gpu), sin=sin.to(gpu), law=law, do_norm=2)
    assert rel_l2(gq[:, :d], ref_of(0, wq)) < 4e-3
    assert torch.equal(gq[:, d:].cpu(), buf[:, d:])


def test_split_launches_equal_one_launch_per_segment(gpu):
    """Joint-block launches over text + image rows (split): the LayerNorm modulations (bf16
    and fused e4m3) and the q/k norm + rope equal one launch per segment, bit for bit. The
    image vectors sit before the text ones in memory (a negative batch stride)."""
    g = torch.Generator().manual_seed(21)
    st, s, d, h = 96, 352, 1024, 8
    x = rnd(g, s, d, std=2.0).to(gpu)
    mod = rnd(g, 1, 4 * d, std=0.3).to(gpu)
    img_sh, img_sc, txt_sh, txt_sc = (mod[:, i * d:(i + 1) * d] for i in range(4))
    one = kernels.layernorm_modulate(x, txt_sc, txt_sh, eps=1e-6, split=st, mul2=img_sc,
                                     add2=img_sh)
    ref = torch.cat([kernels.layernorm_modulate(x[:st], txt_sc, txt_sh, eps=1e-6),
                     kernels.layernorm_modulate(x[st:], img_sc, img_sh, eps=1e-6)])
    assert torch.equal(one.view(torch.int16), ref.view(torch.int16))
    q1, s1 = kernels.layernorm_modulate_fp8(x, txt_sc, txt_sh, eps=1e-6, split=st,
                                            mul2=img_sc, add2=img_sh)
    qa, sa = kernels.layernorm_modulate_fp8(x[:st], txt_sc, txt_sh, eps=1e-6)
    qb, sb = kernels.layernorm_modulate_fp8(x[st:], img_sc, img_sh, eps=1e-6)
    assert torch.equal(q1.view(torch.uint8), torch.cat([qa, qb]).view(torch.uint8))
    assert torch.equal(s1, torch.cat([sa, sb]))
    buf = rnd(g, s, 3 * h * 128).to(gpu)
    w = [(1 + 0.1 * torch.randn(128, generator=g)).bfloat16().to(gpu) for _ in range(4)]
    cos, sin = (torch.randn(s, 128, generator=g).to(gpu) for _ in range(2))
    b1, b2 = buf.clone(), buf.clone()
    kw = dict(heads=h, head_dim=128, q_off=0, k_off=h * 128, eps=1e-6, law=0)
    kernels.qk_norm_rope(b1, wq=w[0], wk=w[1], cos=cos, sin=sin, split=st, wq2=w[2], wk2=w[3],
                         **kw)
    kernels.qk_norm_rope(b2[:st], wq=w[0], wk=w[1], cos=cos[:st], sin=sin[:st], **kw)
    kernels.qk_norm_rope(b2[st:], wq=w[2], wk=w[3], cos=cos[st:], sin=sin[st:], **kw)
    assert torch.equal(b1.view(torch.int16), b2.view(torch.int16))


@pytest.mark.parametrize("law", [0, 1])
def test_rope_laws(gpu, law):
    g = torch.Generator().manual_seed(11 + law)
    x = rnd(g, 2, 3, 50, 128, dtype=torch.float32)
    cos = torch.randn(50, 128, generator=g)
    sin = torch.randn(50, 128, generator=g)  # not repeat-interleaved: the laws differ
    fn = ops.apply_rotary_emb_fp32 if law == 0 else ops.apply_rotary_emb
    ref = fn(x, cos, sin)
    out = kernels.rope(x.to(gpu), cos.to(gpu), sin.to(gpu), law=law)
    assert rel_l2(out, ref) < 1e-6


@pytest.mark.parametrize("m,k,n,xdt", [(1, 256, 3072, torch.bfloat16), (1, 3072, 1001, torch.bfloat16),
                                        (2, 5120, 777, torch.bfloat16), (2, 6656, 301, torch.float32),
                                        (8, 1536, 64, torch.bfloat16), (1, 3072, 7, torch.float32)])
def test_gemv_shapes_tail_and_strided_weights(gpu, m, k, n, xdt):
    """Whole 3072-wide groups, the guarded tail after them (k = 256, 5120, 6656, 1536), column
    counts that leave the last wave's second column out of range, and a weight view whose row
    stride exceeds k."""
    print(f"gemv m={m} k={k} n={n} {xdt}", flush=True)
    g = torch.Generator().manual_seed(k + n)
    xv = rnd(g, m, k).to(xdt)
    wfull = rnd(g, n, k + 64, std=0.02)
    w = wfull[:, 32:32 + k]
    b = rnd(g, n, std=0.1)
    for act in (0, 1):
        xin = torch.nn.functional.silu(xv.float()).to(xdt).float() if act else xv.float()
        ref = ops.linear(xin, w.float(), b.float())
        out = kernels.gemv(xv.to(gpu), wfull.to(gpu)[:, 32:32 + k], b.to(gpu), act=act)
        assert out.dtype == xdt
        assert rel_l2(out, ref) < (4e-3 if xdt == torch.bfloat16 else 1e-5)
    if m == 8:  # m rounds up to an 8-row LDS stage: 8 * k must stay within 16384
        with pytest.raises(NotImplementedError):
            kernels.gemv(torch.zeros(8, 2056, device=gpu), w.to(gpu)[:, :8].repeat(1, 257))


def test_bf16_rounding_every_upper_half_and_midpoint(gpu):
    """Kernels round fp32 results to bf16 to nearest even: LN(x) * 0 + add with fp32 add vectors
    returns bf16(add) exactly. Every upper half-word with the low halves that decide the rounding
    (0, below the tie, the tie, above it, all ones, one random) against torch's rounding, bit for
    bit; NaN stays NaN (torch writes one canonical NaN, the kernels keep the payload)."""
    g = torch.Generator().manual_seed(5)
    hi = torch.arange(65536, dtype=torch.int64) << 16
    lows = [torch.full((65536,), lo, dtype=torch.int64) for lo in (0, 0x7fff, 0x8000, 0x8001, 0xffff)]
    lows.append(torch.randint(0, 65536, (65536,), generator=g, dtype=torch.int64))
    bits = torch.cat([hi | lo for lo in lows])
    vals = torch.where(bits >= 2**31, bits - 2**32, bits).to(torch.int32).view(torch.float32)
    dim = 8192
    add = vals.reshape(-1, dim)
    rows = add.shape[0]
    x = torch.randn(rows, dim, generator=g)
    out = kernels.layernorm_modulate(x.to(gpu), torch.zeros(rows, dim, device=gpu), add.to(gpu),
                                     eps=1e-6, one_plus=False, out_dtype=torch.bfloat16,
                                     rows_per_batch=1).cpu().reshape(-1)
    ref = vals.bfloat16()
    nan = torch.isnan(vals)
    assert torch.isnan(out[nan]).all()
    got, want = out[~nan].view(torch.int16), ref[~nan].view(torch.int16)
    zero = vals[~nan] == 0  # LN(x) * 0 + (-0) may be +0
    assert torch.equal(got[~zero], want[~zero])
    assert (out[~nan][zero] == 0).all()


def test_gelu_gate_residual_gemv_timestep(gpu):
    g = torch.Generator().manual_seed(12)
    x = rnd(g, 1001, dtype=torch.float32) * 4
    assert rel_l2(kernels.gelu_tanh(x.to(gpu)), ops.gelu_tanh(x)) < 1e-5
    r, y, gt = rnd(g, 64, 256), rnd(g, 64, 256), rnd(g, 256)
    out = kernels.gate_residual(r.to(gpu), y.to(gpu), gt.to(gpu))
    assert rel_l2(out, r.float() + gt.float() * y.float()) < 4e-3
    for m in (1, 2, 3):
        xv = rnd(g, m, 3072)
        w = rnd(g, 1000, 3072, std=0.02)
        b = rnd(g, 1000, std=0.1)
        silu_x = torch.nn.functional.silu(xv.float()).bfloat16().float()
        ref = ops.linear(silu_x, w.float(), b.float())
        out = kernels.gemv(xv.to(gpu), w.to(gpu), b.to(gpu), act=1)
        assert rel_l2(out, ref) < 4e-3
    t = torch.tensor([0.0, 1.5, 999.0, 437.25])
    ref = ops.timestep_embedding(t, 256, flip_sin_to_cos=True, downscale_freq_shift=0)
    out = kernels.timestep_embedding(t.to(gpu), 256, flip_sin_to_cos=True,
                                     downscale_freq_shift=0.0)
    assert (out.cpu() - ref).abs().max().item() < 2e-4


def test_attention_matches_the_reference_cpu_op_vectors(gpu):
    """The HIP kernel on the bf16 inputs the reference CPU attention op was run on
    (tests/golden/attention_reference.json): every contract form within bf16 rounding of the
    reference's own bf16 output (it rounds scores and probabilities to bf16; the kernel keeps
    them in fp32)."""
    import json
    from pathlib import Path

    from tests.golden.make_attention_golden import cases, decode

    g = json.loads((Path(__file__).parent / "golden" / "attention_reference.json").read_text())
    for name, ((q, k, v), kw) in cases(torch.bfloat16).items():
        print(f"attention vs reference vectors: {name}", flush=True)
        kw = {key: (val.to(gpu) if torch.is_tensor(val) else val) for key, val in kw.items()}
        if "scale" not in kw:
            kw["scale"] = 1.0  # the contract's scale=None
        out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), **kw)
        torch.cuda.synchronize()
        want = decode(g[f"{name}.bfloat16"])
        assert tuple(out.shape) == tuple(want.shape), name
        e = rel_l2(out, want)
        print(f"  rel L2 {e:.3e}", flush=True)
        assert e < 2e-2, name


def test_attention_fp32_matches_the_reference_cpu_op_vectors(gpu):
    """fp32 inputs run the fp32 kernel: every contract form against the reference CPU op's own
    fp32 output (tests/golden/attention_reference.json), to fp32 summation-order error."""
    import json
    from pathlib import Path

    from tests.golden.make_attention_golden import cases, decode

    g = json.loads((Path(__file__).parent / "golden" / "attention_reference.json").read_text())
    for name, ((q, k, v), kw) in cases(torch.float32).items():
        print(f"fp32 attention vs reference vectors: {name}", flush=True)
        kw = {key: (val.to(gpu) if torch.is_tensor(val) else val) for key, val in kw.items()}
        kw.setdefault("scale", 1.0)
        out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), **kw)
        torch.cuda.synchronize()
        want = decode(g[f"{name}.float32"])
        assert out.dtype == torch.float32 and tuple(out.shape) == tuple(want.shape), name
        e = rel_l2(out, want)
        assert e < 1e-5, f"{name}: rel L2 {e:.3e}"


# the T5 / UMT5 text encoders' attention: head_dim 64, unscaled scores plus a relative-position
# bias (an additive [1, H, S, S] mask), key padding as a bool mask; ragged query/key counts
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("b,h,sq,sk", [(1, 2, 1, 1), (2, 3, 77, 77), (1, 4, 512, 512),
                                       (1, 2, 300, 1100)])
def test_attention_head_dims_and_fp32(gpu, dtype, d, b, h, sq, sk):
    print(f"attention d={d} {dtype} b={b} h={h} sq={sq} sk={sk}", flush=True)
    g = torch.Generator().manual_seed(d + sq + sk)
    q, k, v = _attn_case(g, b, h, sq, sk, d=d, dtype=dtype)
    qf, kf, vf = q.float(), k.float(), v.float()
    tol = 2e-5 if dtype == torch.float32 else 1e-2
    s = 1 / math.sqrt(d)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=s)
    assert out.dtype == dtype and out.shape == q.shape
    assert rel_l2(out, ops.attention(qf, kf, vf, scale=s)) < tol
    bias = torch.randn(1, h, sq, sk, generator=g) * 3.0
    ref = ops.attention(qf, kf, vf, scale=1.0, attention_mask=bias)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=1.0,
                            attention_mask=bias.to(gpu))
    assert rel_l2(out, ref) < tol
    keep = torch.ones(b, 1, 1, sk, dtype=torch.bool)
    keep[..., sk - sk // 3:] = False
    keep[..., 0] = True
    ref = ops.attention(qf, kf, vf, scale=s, attention_mask=keep)
    out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=s, attention_mask=keep.to(gpu))
    assert rel_l2(out, ref) < tol
    if sq == sk:
        ref = ops.attention(qf, kf, vf, scale=s, causal=True)
        out = kernels.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=s, causal=True)
        assert rel_l2(out, ref) < tol


def test_attention_fp32_bounds_strides_and_empty_windows(gpu):
    """The fp32 kernel on column views of one [S, 3 H D] buffer with per-query key windows, an
    empty window averaging v."""
    g = torch.Generator().manual_seed(31)
    s, h, d = 333, 3, 64
    buf = torch.randn(s, 3 * h * d, generator=g)
    views = [buf[:, i * h * d:(i + 1) * h * d].reshape(s, h, d).transpose(0, 1) for i in range(3)]
    bmin = torch.randint(0, 100, (h, s, 1), generator=g, dtype=torch.int32)
    bmax = bmin + torch.randint(1, 200, (h, s, 1), generator=g, dtype=torch.int32)
    bmax[1, :7] = bmin[1, :7]
    ref = ops.attention(*views, scale=0.1, bound_min=bmin, bound_max=bmax)
    gb = buf.to(gpu)
    gv = [gb[:, i * h * d:(i + 1) * h * d].reshape(s, h, d).transpose(0, 1) for i in range(3)]
    out = kernels.attention(*gv, scale=0.1, bound_min=bmin.to(gpu), bound_max=bmax.to(gpu))
    assert rel_l2(out, ref) < 2e-5
    assert rel_l2(out[1, :7].cpu(), views[2][1].mean(dim=0).expand(7, -1)) < 2e-5
