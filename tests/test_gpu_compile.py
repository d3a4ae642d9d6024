"""torch.compile over the rocm op modules on the GPU: a FLUX-single-block-shaped module built from
the op modules (LayerNorm, linears, RMSNorm, rotary embedding, attention, GELU) traces with
fullgraph=True, its graph holds the HIP kernels as ``difflet_rocm::*`` nodes, and the compiled
output matches the eager one. Also with per-channel fp8 twins, and through the per-block
compile helper the GPU component uses."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from difflet_amd.backends.rocm import compile as rc
from difflet_amd.backends.rocm.ops_impl.attention import attention
from difflet_amd.backends.rocm.ops_impl.embeddings import apply_rotary_emb
from difflet_amd.backends.rocm.ops_impl.linear import ColumnParallelLinear, RowParallelLinear
from difflet_amd.backends.rocm.ops_impl.norm import LayerNorm, RMSNorm

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]
D, HEADS, S = 512, 4, 256


class SingleBlock(nn.Module):
    def __init__(self, dev):
        super().__init__()
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.norm = LayerNorm(D, eps=1e-6, elementwise_affine=False)
        self.qkv = ColumnParallelLinear(D, 3 * D, **bf)
        self.mlp = ColumnParallelLinear(D, 4 * D, **bf)
        self.out = RowParallelLinear(5 * D, D, **bf)
        self.norm_q, self.norm_k = RMSNorm(128).to(dev), RMSNorm(128).to(dev)

    def forward(self, x, cos, sin):
        b, s, d = x.shape
        h = self.norm(x)
        q, k, v = self.qkv(h).view(b, s, 3, HEADS, 128).permute(2, 0, 3, 1, 4).unbind(0)
        q = apply_rotary_emb(self.norm_q(q), cos, sin)
        k = apply_rotary_emb(self.norm_k(k), cos, sin)
        o = attention(q, k, v, scale=1.0 / math.sqrt(128)).transpose(1, 2).reshape(b, s, d)
        m = F.gelu(self.mlp(h), approximate="tanh")
        return x + self.out(torch.cat([o, m], dim=-1))


def _inputs(dev):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, S, D, generator=g).to(dev, torch.bfloat16)
    ang = torch.arange(S)[:, None] * torch.exp(-torch.arange(64) / 8.0)[None, :]
    cos = torch.cos(ang).repeat_interleave(2, dim=-1).to(dev)
    sin = torch.sin(ang).repeat_interleave(2, dim=-1).to(dev)
    return x, cos, sin


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def _kernel_nodes(fn, args) -> tuple[set[str], int]:
    graphs = []

    def record(gm, example_inputs):
        graphs.append(gm)
        return gm.forward

    torch._dynamo.reset()
    torch.compile(fn, backend=record, fullgraph=True)(*args)
    names = {str(n.target) for gm in graphs for n in gm.graph.nodes if n.op == "call_function"}
    return {n for n in names if n.startswith("difflet_rocm.")}, len(graphs)


def test_block_compiles_without_graph_breaks(gpu):
    torch.manual_seed(0)
    blk = SingleBlock(gpu).eval()
    args = _inputs(gpu)
    print("explain + record the FX graph", flush=True)
    explain = torch._dynamo.explain(blk)(*args)
    assert explain.graph_break_count == 0, explain.break_reasons
    nodes, ngraphs = _kernel_nodes(blk, args)
    assert ngraphs == 1
    assert nodes == {"difflet_rocm.layer_norm.default", "difflet_rocm.linear.default",
                     "difflet_rocm.rms_norm.default", "difflet_rocm.rope.default",
                     "difflet_rocm.attention.default"}
    with torch.no_grad():
        y0 = blk(*args)
        torch._dynamo.reset()
        print("inductor compile", flush=True)
        y1 = torch.compile(blk, fullgraph=True, mode="default")(*args)
        y2 = torch.compile(blk, fullgraph=True, mode="default")(*args)
    torch.cuda.synchronize()
    assert torch.isfinite(y0.float()).all()
    e = _rel(y1, y0)
    print(f"compiled vs eager rel L2 {e:.2e}", flush=True)
    assert e < 5e-3
    assert torch.equal(y1, y2)


def test_fp8_twin_block_compiles(gpu):
    from difflet_amd.quant.linear import prepare_fp8_kernels_, quantize_module_
    from difflet_amd.quant.spec import RocmQuantSpec

    torch.manual_seed(1)
    blk = SingleBlock(gpu).eval()
    spec = RocmQuantSpec(targets=(r"qkv", r"mlp", r"out"), format="fp8_rowwise")
    assert quantize_module_(blk, spec, from_dense=True) == ["qkv", "mlp", "out"]
    prepare_fp8_kernels_(blk)
    args = _inputs(gpu)
    nodes, ngraphs = _kernel_nodes(blk, args)
    assert ngraphs == 1 and "difflet_rocm.fp8_linear.default" in nodes
    assert "difflet_rocm.linear.default" not in nodes
    with torch.no_grad():
        y0 = blk(*args)
        torch._dynamo.reset()
        y1 = torch.compile(blk, fullgraph=True, mode="default")(*args)
    torch.cuda.synchronize()
    e = _rel(y1, y0)
    print(f"fp8 compiled vs eager rel L2 {e:.2e}", flush=True)
    assert e < 5e-3


def test_compile_repeated_blocks(gpu):
    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.single_transformer_blocks = nn.ModuleList([SingleBlock(gpu) for _ in range(2)])

        def forward(self, x, cos, sin):
            for b in self.single_transformer_blocks:
                x = b(x, cos, sin)
            return x

    torch.manual_seed(2)
    model = Model().eval()
    args = _inputs(gpu)
    with torch.no_grad():
        y0 = model(*args)
        torch._dynamo.reset()
        assert rc.compile_repeated_blocks_(model, mode="default") == 2
        y1 = model(*args)
    torch.cuda.synchronize()
    e = _rel(y1, y0)
    print(f"per-block compiled model vs eager rel L2 {e:.2e}", flush=True)
    assert e < 5e-3


# ------------------------------------------------ compiled FLUX single block vs the oracle
class FluxSingleOnOps(nn.Module):
    """FLUX's single-stream block (difflet/models/flux/modeling_flux.py:696-736) written on the
    rocm op modules: adaLN-Zero-Single from SiLU(temb), LayerNorm, q/k/v and the MLP, per-head
    RMSNorm, the fp32 RoPE law, attention, one proj_out over [attn | mlp], gated residual."""

    def __init__(self, d, heads, mlp, dev):
        super().__init__()
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.heads = heads
        self.norm_linear = ColumnParallelLinear(d, 3 * d, **bf)
        self.norm = LayerNorm(d, eps=1e-6, elementwise_affine=False)
        self.to_q, self.to_k, self.to_v = (ColumnParallelLinear(d, d, **bf) for _ in range(3))
        self.proj_mlp = ColumnParallelLinear(d, mlp, **bf)
        self.norm_q, self.norm_k = RMSNorm(128).to(dev), RMSNorm(128).to(dev)
        self.proj_out = RowParallelLinear(d + mlp, d, **bf)

    def load_oracle(self, w):
        names = {"norm_linear": "norm.linear", "to_q": "attn.to_q", "to_k": "attn.to_k",
                 "to_v": "attn.to_v", "proj_mlp": "proj_mlp", "proj_out": "proj_out"}
        with torch.no_grad():
            for mine, theirs in names.items():
                getattr(self, mine).weight.copy_(w[f"{theirs}.weight"])
                getattr(self, mine).bias.copy_(w[f"{theirs}.bias"])
            self.norm_q.weight.copy_(w["attn.norm_q.weight"])
            self.norm_k.weight.copy_(w["attn.norm_k.weight"])

    def forward(self, x, temb, cos, sin):
        from difflet_amd.backends.rocm.ops_impl.embeddings import apply_rotary_emb_fp32

        b, s, d = x.shape
        shift, scale, gate = self.norm_linear(F.silu(temb)).chunk(3, dim=1)
        nh = self.norm(x) * (1 + scale[:, None]) + shift[:, None]
        mlp = F.gelu(self.proj_mlp(nh), approximate="tanh")
        heads = lambda t: t.view(b, s, self.heads, 128).transpose(1, 2)  # noqa: E731
        q = apply_rotary_emb_fp32(self.norm_q(heads(self.to_q(nh))), cos, sin)
        k = apply_rotary_emb_fp32(self.norm_k(heads(self.to_k(nh))), cos, sin)
        o = attention(q, k, heads(self.to_v(nh)), scale=1.0 / math.sqrt(128))
        o = o.transpose(1, 2).reshape(b, s, d)
        return x + gate[:, None] * self.proj_out(torch.cat([o, mlp], dim=-1))


@pytest.mark.parametrize("kind", ["bf16", "fp8"])
def test_compiled_flux_single_block_matches_the_oracle(gpu, kind, parity):
    """The compiled op-module block at FLUX width (3072, 24 heads, MLP 12288) on 128 + 16 x 16
    tokens against oracle.flux.single_block on the same weights: rel L2 <= 1e-2 against the
    fp32 block (bf16), <= 3e-2 against the oracle of the per-channel fp8 law with bf16
    activations (fp8 twins on every linear but the adaLN one)."""
    from difflet_amd.quant.linear import prepare_fp8_kernels_, quantize_module_
    from difflet_amd.quant.spec import RocmQuantSpec
    from oracle import flux as oflux
    from oracle import ops

    shape = oflux.FluxShape(n_double=1, n_single=1)
    w = oflux.single_block_weights(shape, 5, 0)
    g = torch.Generator().manual_seed(5)
    st, hw = 128, (16, 16)
    s = st + hw[0] * hw[1]
    x = torch.randn(1, s, shape.hidden, generator=g).bfloat16().float()
    temb = torch.randn(1, shape.hidden, generator=g).bfloat16().float()
    cos, sin = ops.flux_pos_embed(ops.flux_ids(st, *hw))
    blk = FluxSingleOnOps(shape.hidden, shape.heads, shape.mlp, gpu).eval()
    blk.load_oracle(w)
    if kind == "fp8":
        spec = RocmQuantSpec(targets=(r"to_q", r"to_k", r"to_v", r"proj_mlp", r"proj_out"),
                             format="fp8_rowwise")
        assert len(quantize_module_(blk, spec, from_dense=True)) == 5
        prepare_fp8_kernels_(blk)
    args = (x.to(gpu, torch.bfloat16), temb.to(gpu, torch.bfloat16), cos.to(gpu), sin.to(gpu))
    print(f"compiled FLUX single block ({kind}) vs oracle", flush=True)
    with torch.no_grad():
        torch._dynamo.reset()
        y = torch.compile(blk, fullgraph=True, mode="default")(*args)
        mods = blk.norm_linear(F.silu(args[1])).float().cpu()
    torch.cuda.synchronize()
    full = oflux.single_block(w, x, temb, cos, sin, shape)
    if kind == "bf16":
        e = _rel(y.cpu(), full)
        print(f"compiled bf16 block vs fp32 oracle rel L2 {e:.3e}", flush=True)
        parity("compiled op-module single block, rel L2 vs fp32 oracle", e, 1e-2)
        assert e < 1e-2
        return
    ref = oflux.single_block(w, x, temb, cos, sin, shape, quant="fp8", act_dtype=torch.bfloat16,
                             store=torch.bfloat16, mods=mods)
    e, fmt_dev, fmt_ref = _rel(y.cpu(), ref), _rel(y.cpu(), full), _rel(ref, full)
    print(f"compiled fp8 block vs same-law oracle rel L2 {e:.3e}; format error device "
          f"{fmt_dev:.3e}, oracle {fmt_ref:.3e}", flush=True)
    parity("compiled op-module single block fp8, rel L2 vs same-law oracle", e, 3e-2)
    assert e < 3e-2
    assert abs(fmt_dev - fmt_ref) < 0.1 * fmt_ref
