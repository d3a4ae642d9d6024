"""The rocm backend's op surface and quantized linears on the GPU against the oracle."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fp8 as ofp8
from oracle import mx as omx
from oracle import ops

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return ((a - b).norm() / b.norm()).item()


def test_ops_attention_forms(gpu):
    from difflet_amd.backends.rocm.ops_impl import attention as A

    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 3, 100, 128, generator=g).bfloat16() for _ in range(3))
    qf, kf, vf = q.float(), k.float(), v.float()
    sc = 1 / math.sqrt(128)
    ref = ops.attention(qf, kf, vf, scale=sc)
    assert rel_l2(A.attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=sc), ref) < 1e-2
    folded = A.attention(q.reshape(6, 100, 128).to(gpu), k.reshape(6, 100, 128).to(gpu),
                         v.reshape(6, 100, 128).to(gpu), scale=sc, tp_q=True, tp_k=True)
    assert folded.shape == (6, 100, 128) and rel_l2(folded.reshape(ref.shape), ref) < 1e-2
    assert rel_l2(A.cross_attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=sc, tp_q=True), ref) < 1e-2
    assert rel_l2(A.ring_attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=sc), ref) < 1e-2
    assert rel_l2(A.ulysses_attention(q.to(gpu), k.to(gpu), v.to(gpu), scale=sc), ref) < 1e-2
    # joint forms: keys [image | text], right-padded text masked by its valid length
    ik, iv, tk, tv = kf[:, :, :70], vf[:, :, :70], kf[:, :, 70:], vf[:, :, 70:]
    valid = torch.tensor([20, 30])
    keys = torch.cat([ik, tk], dim=2)
    vals = torch.cat([iv, tv], dim=2)
    bmax = (70 + valid).view(2, 1, 1, 1).expand(2, 3, 100, 1)
    ref_j = ops.attention(qf, keys, vals, scale=sc, bound_min=torch.zeros_like(bmax), bound_max=bmax)
    G = lambda t: t.bfloat16().to(gpu)  # noqa: E731
    out = A.joint_ring_attention(q.to(gpu), G(ik), G(iv), G(tk), G(tv), scale=sc,
                                 text_valid_len=valid.to(gpu))
    assert rel_l2(out, ref_j) < 1e-2
    oi, ot = A.joint_ulysses_attention(q[:, :, :60].to(gpu), q[:, :, 60:].to(gpu), G(ik), G(iv),
                                       G(tk), G(tv), scale=sc)
    ref_u = ops.attention(qf, keys, vals, scale=sc)
    assert rel_l2(torch.cat([oi, ot], dim=2), ref_u) < 1e-2
    with pytest.raises(NotImplementedError):
        A.attention(q.double().to(gpu), k.double().to(gpu), v.double().to(gpu))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d", [32, 40, 80, 96, 120])
def test_ops_attention_other_head_dims(gpu, dtype, d):
    """head_dim other than 64 / 128 (the reference op takes any): q, k, v zero-padded to the
    kernel's width, the output cut back, against the fp32 attention of the oracle, with a bool
    mask, per-query bounds and causal masking too; the scale is the caller's."""
    from difflet_amd.backends.rocm.ops_impl import attention as A

    print(f"attention head_dim {d} {dtype}", flush=True)
    g = torch.Generator().manual_seed(d)
    q, k, v = (torch.randn(2, 3, 150, d, generator=g).to(dtype) for _ in range(3))
    qf, kf, vf = q.float(), k.float(), v.float()
    sc = 1 / math.sqrt(d)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    G = lambda t: t.to(gpu)  # noqa: E731
    out = A.attention(G(q), G(k), G(v), scale=sc)
    assert out.shape == q.shape and out.dtype == dtype
    assert rel_l2(out, ops.attention(qf, kf, vf, scale=sc)) < tol
    mask = torch.rand(2, 1, 150, 150, generator=g) > 0.3
    assert rel_l2(A.attention(G(q), G(k), G(v), scale=sc, attention_mask=G(mask)),
                  ops.attention(qf, kf, vf, scale=sc, attention_mask=mask)) < tol
    lo = torch.randint(0, 40, (2, 3, 150, 1), generator=g)
    hi = lo + torch.randint(1, 110, (2, 3, 150, 1), generator=g)
    assert rel_l2(A.attention(G(q), G(k), G(v), scale=sc, bound_min=G(lo.int()), bound_max=G(hi.int())),
                  ops.attention(qf, kf, vf, scale=sc, bound_min=lo, bound_max=hi)) < tol
    assert rel_l2(A.attention(G(q), G(k), G(v), scale=sc, causal=True),
                  ops.attention(qf, kf, vf, scale=sc, causal=True)) < tol
    with pytest.raises(NotImplementedError):
        A.attention(G(q.new_zeros(1, 1, 4, 160)), G(q.new_zeros(1, 1, 4, 160)),
                    G(q.new_zeros(1, 1, 4, 160)))


@pytest.mark.parametrize("m,k,n", [(3, 3072, 500), (300, 256, 128), (77, 100, 30)])
def test_ops_linear_modules(gpu, m, k, n):
    from difflet_amd.backends.rocm.ops_impl import linear as L

    g = torch.Generator().manual_seed(m + k)
    x = torch.randn(2, m, k, generator=g).bfloat16()
    col = L.ColumnParallelLinear(k, n, bias=True, gather_output=False, dtype=torch.bfloat16)
    row = L.RowParallelLinear(k, n, bias=True, skip_bias_add=True, dtype=torch.bfloat16)
    with torch.no_grad():
        for mod in (col, row):
            mod.weight.copy_(torch.randn(n, k, generator=g) * 0.05)
            mod.bias.copy_(torch.randn(n, generator=g) * 0.1)
    ref = F.linear(x.float(), col.weight.float(), col.bias.float())
    col, row = col.to(gpu), row.to(gpu)
    out = col(x.to(gpu))
    assert out.shape == (2, m, n) and rel_l2(out, ref) < 4e-3
    y, b = row(x.to(gpu))
    assert b is row.bias
    assert rel_l2(y, F.linear(x.float(), row.weight.float().cpu())) < 4e-3


@pytest.mark.parametrize("m,k,n", [(3, 3072, 500), (300, 256, 128), (77, 100, 30), (512, 4096, 10240)])
def test_ops_linear_modules_fp32_weights(gpu, m, k, n):
    """fp32 weights run the fp32 GEMM (K / N off multiples of 4 padded on the weight), fp32
    math as F.linear does."""
    from difflet_amd.backends.rocm.ops_impl import linear as L

    g = torch.Generator().manual_seed(m + k + 1)
    x = torch.randn(2, m, k, generator=g)
    col = L.ColumnParallelLinear(k, n, bias=True, gather_output=False, dtype=torch.float32)
    row = L.RowParallelLinear(k, n, bias=False, skip_bias_add=True, dtype=torch.float32)
    ref = F.linear(x.double(), col.weight.double(), col.bias.double())
    col, row = col.to(gpu), row.to(gpu)
    out = col(x.to(gpu))
    assert out.dtype == torch.float32 and out.shape == (2, m, n)
    assert rel_l2(out, ref) < 1e-5
    y, b = row(x.to(gpu))
    assert b is None
    assert rel_l2(y, F.linear(x.double(), row.weight.double().cpu())) < 1e-5


def test_ops_norms_and_rotary(gpu):
    from difflet_amd.backends.rocm.ops_impl import embeddings as E
    from difflet_amd.backends.rocm.ops_impl import norm as N

    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 50, 3072, generator=g).bfloat16()
    rms = N.RMSNorm(3072)
    with torch.no_grad():
        rms.weight.copy_(torch.rand(3072, generator=g) + 0.5)
    assert rel_l2(rms.to(gpu)(x.to(gpu)), ops.rms_norm_fp32(x.float(), rms.weight.cpu().float(), 1e-6)) < 4e-3
    ln = N.LayerNorm(3072, eps=1e-6)
    with torch.no_grad():
        ln.weight.copy_(torch.randn(3072, generator=g))
        ln.bias.copy_(torch.randn(3072, generator=g))
    ref = F.layer_norm(x.float(), (3072,), ln.weight, ln.bias, eps=1e-6)
    assert rel_l2(ln.to(gpu)(x.to(gpu)), ref) < 4e-3
    # rotary: [B, H, S, D] with [S, D] tables, and [B, S, H, D] with [1, S, 1, D] tables
    xr = torch.randn(2, 4, 60, 128, generator=g).bfloat16()
    cos, sin = torch.randn(60, 128, generator=g), torch.randn(60, 128, generator=g)
    assert rel_l2(E.apply_rotary_emb_fp32(xr.to(gpu), cos.to(gpu), sin.to(gpu)),
                  ops.apply_rotary_emb_fp32(xr.float(), cos, sin)) < 4e-3
    xs = xr.transpose(1, 2).contiguous()
    out = E.apply_rotary_emb(xs.to(gpu), cos[None, :, None].to(gpu), sin[None, :, None].to(gpu))
    ref = ops.apply_rotary_emb(xs.float(), cos[None, :, None], sin[None, :, None])
    assert out.shape == xs.shape and rel_l2(out, ref) < 4e-3


@pytest.mark.parametrize("fmt", ["fp8_rowwise", "mxfp8"])
def test_quantized_linear_twins(gpu, fmt):
    from difflet_amd.backends.rocm.ops_impl import linear as L
    from difflet_amd.quant import linear as Q
    from difflet_amd.quant.spec import RocmQuantSpec

    g = torch.Generator().manual_seed(2)
    k, n = 384, 256
    m = torch.nn.Module()
    m.to_q = L.ColumnParallelLinear(k, n, bias=True, gather_output=False, dtype=torch.bfloat16)
    m.to_k = L.ColumnParallelLinear(k, n, bias=True, gather_output=False, dtype=torch.bfloat16)
    m.to_v = L.ColumnParallelLinear(k, n, bias=True, gather_output=False, dtype=torch.bfloat16)
    with torch.no_grad():
        for mod in (m.to_q, m.to_k, m.to_v):
            mod.weight.copy_(torch.randn(n, k, generator=g) * 0.05)
            mod.bias.copy_(torch.randn(n, generator=g) * 0.1)
    dense = {nm: (getattr(m, nm).weight.detach().float().clone(),
                  getattr(m, nm).bias.detach().float().clone()) for nm in ("to_q", "to_k", "to_v")}
    m = m.to(gpu)
    names = Q.quantize_module_(m, RocmQuantSpec(targets=(r"to_(q|k|v)",), format=fmt),
                               from_dense=True)
    assert names == ["to_q", "to_k", "to_v"]
    # stored codes and scales are the oracle's law, bit for bit
    w, _ = dense["to_q"]
    if fmt == "mxfp8":
        q_ref, s_ref = omx.quantize_mx(w.numpy())
    else:
        q_ref, s_ref = ofp8.quantize_rowwise(w.numpy())
    assert np.array_equal(m.to_q.weight.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.array_equal(m.to_q.weight_scale.cpu().numpy(), s_ref)
    x = torch.randn(3, 70, k, generator=g).bfloat16()
    Q.prepare_fp8_kernels_(m, fuse=True)
    assert hasattr(m, "fused_qkv")
    for nm in ("to_q", "to_v"):
        wd, bd = dense[nm]
        wq, ws = (omx.quantize_mx(wd.numpy()) if fmt == "mxfp8" else ofp8.quantize_rowwise(wd.numpy()))
        lin = omx.mx_linear if fmt == "mxfp8" else ofp8.fp8_linear
        ref = torch.from_numpy(lin(x.float().numpy().reshape(-1, k), wq, ws, bd.numpy())).reshape(3, 70, n)
        assert rel_l2(getattr(m, nm)(x.to(gpu)), ref) < 4e-3
    fq, fk, fv = m.fused_qkv(x.to(gpu))
    assert torch.equal(fq, m.to_q(x.to(gpu))) and torch.equal(fv, m.to_v(x.to(gpu)))
