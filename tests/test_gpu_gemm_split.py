"""GEMMs whose tiles are cut along K over the compute units (the split schedule that runs when
the last wave of whole tiles would be poorly filled): the same results as whole tiles, the fp32
reference within bf16 output rounding, bit-identical reruns, and a workspace left zeroed."""

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


def rnd(g, *shape, std=1.0):
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def _operands(kind, a, w, gpu):
    if kind == "bf16":
        return a.to(gpu), w.to(gpu), None, None
    if kind == "fp8":
        aq, sa = kernels.quantize_fp8_rowwise(a.to(gpu))
        wq, sw = kernels.quantize_fp8_rowwise(w.to(gpu))
        return aq, wq, sa, sw
    aq, sa = kernels.quantize_mxfp8(a.to(gpu), swizzled=True)
    wq, sw = kernels.quantize_mxfp8(w.to(gpu), swizzled=True)
    return aq, wq, sa, sw


def _reference(kind, a, w, b):
    if kind == "bf16":
        return ops.linear(a.float(), w.float(), b.float())
    if kind == "fp8":
        wq, ws = ofp8.quantize_rowwise(w.float().numpy())
        return torch.from_numpy(ofp8.fp8_linear(a.float().numpy(), wq, ws, b.float().numpy()))
    wq, ws = omx.quantize_mx(w.float().numpy())
    return torch.from_numpy(omx.mx_linear(a.float().numpy(), wq, ws, b.float().numpy()))


# (m, n, k): 336 and 360 tiles (a wave of whole tiles, then the last 80 / 104 cut in groups of
# 32 over the 8 XCDs, one or two XCDs per tile; k = 6144 so that every kind's cut saves the
# planner's minimum of 24 K stages), 15 tiles of a long K (one group cut over all 8 XCDs:
# eight contributors per tile)
SHAPES = [(7168, 3072, 6144), (4608, 5120, 6144), (600, 1280, 8192)]


@pytest.mark.parametrize("kind", ["bf16", "fp8", "mx"])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_split_gemm_equals_whole_tiles_and_reference(gpu, kind, m, n, k):
    print(f"split gemm {kind} m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
    aq, wq, sa, sw = _operands(kind, a, w, gpu)
    bg = b.to(gpu)
    outs = []
    for ws in ("shared", "shared", None):
        c = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        kernels.gemm_grouped([kernels.Problem(aq, wq, c, bg, a_scale=sa, w_scale=sw)],
                             kind=kind, workspace=ws)
        outs.append(c)
    torch.cuda.synchronize()
    split1, split2, whole = outs
    assert torch.equal(split1.view(torch.int16), split2.view(torch.int16))  # deterministic
    assert not torch.isnan(split1).any()
    # fp32 partial sums in another order: at most a bf16 rounding step apart
    assert rel_l2(split1, whole) < 2e-3
    assert rel_l2(split1, _reference(kind, a, w, b)) < 4e-3
    ctr = kernels.gemm_workspace(torch.device(gpu))[:16384].view(torch.int32)
    assert int(torch.count_nonzero(ctr)) == 0  # every counter back at zero


# MXFP8 cuts K in units of 4 stages (one E8M0 block per row of 128 K); these K leave a shorter
# last unit: 6912 = 54 stages at 336 tiles (the last unit 2 stages), 7808 = 61 stages on 15
# tiles (the last unit 1 stage, eight contributors per tile). Both plans split (test_abi.py).
@pytest.mark.parametrize("m,n,k", [(7168, 3072, 6912), (600, 1280, 7808)])
def test_split_gemm_mx_with_a_short_last_unit(gpu, m, n, k):
    test_split_gemm_equals_whole_tiles_and_reference(gpu, "mx", m, n, k)


@pytest.mark.parametrize("kind", ["bf16", "fp8", "mx"])
def test_split_gemm_gate_residual_in_place_grouped(gpu, kind):
    """Qwen-Image's output projection shape: text and image problems in one launch (1 + 27
    row tiles x 12 = 336 tiles, the last 80 cut), gate * (acc + bias) + residual written over
    the residual. MXFP8 runs this epilogue on the split in the Qwen-Image step's FF2. fp8 and
    MXFP8 take K = 6144: at 3072 their cut saves under the planner's 24 stages."""
    g = torch.Generator().manual_seed(11)
    n, k = 3072, 3072 if kind == "bf16" else 6144
    probs, refs = [], []
    for m in (256, 6889):
        a, w, b = rnd(g, m, k), rnd(g, n, k, std=0.05), rnd(g, n, std=0.1)
        gate, res = rnd(g, 1, n), rnd(g, m, n)
        aq, wq, sa, sw = _operands(kind, a, w, gpu)
        r = res.to(gpu)
        probs.append(kernels.Problem(aq, wq, r, b.to(gpu), gate.to(gpu), r, a_scale=sa,
                                     w_scale=sw))
        refs.append((r, res.float() + gate.float() * _reference(kind, a, w, b)))
    kernels.gemm_grouped(probs, kind=kind, epilogue=_lib.EPI_GATE_RESIDUAL, workspace="shared")
    torch.cuda.synchronize()
    for r, ref in refs:
        assert rel_l2(r, ref) < 4e-3
