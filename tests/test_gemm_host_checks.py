"""The GEMM's host-side refusals, on the CPU: every vector the kernel reads beside A and W
(bias, gate, residual, fp8 / MXFP8 scales, q/k norm weights, RoPE rows) is checked for dtype and
extent before any device work, since the kernel indexes them without bounds checks."""

import ctypes

import pytest
import torch

from difflet_amd import _lib, kernels
from difflet_amd.kernels import Problem, QkNormRope

M, N, K = 300, 512, 256
DEVICE_MSG = "rocm kernels take device tensors"  # validation passed, only the device is wrong


def _bf16(*shape):
    return torch.zeros(shape, dtype=torch.bfloat16)


def _prob(kind="bf16", **kw):
    if kind == "bf16":
        a, w = _bf16(M, K), _bf16(N, K)
    else:
        a = torch.zeros(M, K, dtype=torch.float8_e4m3fn)
        w = torch.zeros(N, K, dtype=torch.float8_e4m3fn)
    if kind == "fp8":
        kw.setdefault("a_scale", torch.ones(M))
        kw.setdefault("w_scale", torch.ones(N))
    if kind == "mx":
        kw.setdefault("a_scale", torch.zeros(M, K // 32, dtype=torch.uint8))
        kw.setdefault("w_scale", torch.zeros(N, K // 32, dtype=torch.uint8))
    return Problem(a, w, _bf16(M, N), **kw)


def _run(p, kind="bf16", epilogue=_lib.EPI_NONE, qk=None):
    kernels.gemm_grouped([p], kind=kind, epilogue=epilogue, qk=qk)


def _gated(**kw):
    kw.setdefault("gate", _bf16(1, N))
    kw.setdefault("residual", _bf16(M, N))
    return _prob(**kw)


@pytest.mark.parametrize("kind", ["bf16", "fp8", "mx"])
def test_well_formed_problems_reach_the_device_check(kind):
    with pytest.raises(ValueError, match=DEVICE_MSG):
        _run(_prob(kind, bias=_bf16(N)), kind)
    with pytest.raises(ValueError, match=DEVICE_MSG):
        _run(_gated(kind=kind), kind, _lib.EPI_GATE_RESIDUAL)


@pytest.mark.parametrize("make, kind, epi, exc, msg", [
    (lambda: _prob(bias=_bf16(N - 4)), "bf16", _lib.EPI_NONE, ValueError, "bias must be"),
    (lambda: _prob(bias=torch.zeros(N)), "bf16", _lib.EPI_NONE, TypeError, "bias must be"),
    (lambda: _prob(bias=_bf16(2 * N)[::2]), "bf16", _lib.EPI_NONE, ValueError, "bias must be"),
    (lambda: _prob(gate=_bf16(1, N)), "bf16", _lib.EPI_GATE_RESIDUAL, ValueError,
     "needs gate and residual"),
    (lambda: _gated(gate=_bf16(N - 4)), "bf16", _lib.EPI_GATE_RESIDUAL, ValueError,
     "gate must hold"),
    (lambda: _gated(gate=torch.zeros(1, N)), "bf16", _lib.EPI_GATE_RESIDUAL, TypeError,
     "gate must be bf16"),
    # two batch elements of 256 rows (M = 300) need two gate rows
    (lambda: _gated(gate=_bf16(1, N), rows_per_batch=256), "bf16", _lib.EPI_GATE_RESIDUAL,
     ValueError, r"gate must hold 2 row"),
    (lambda: _gated(residual=_bf16(M - 1, N)), "bf16", _lib.EPI_GATE_RESIDUAL, ValueError,
     "residual must be"),
    (lambda: _gated(residual=_bf16(M, N - 4)), "bf16", _lib.EPI_GATE_RESIDUAL, ValueError,
     "residual must be"),
    (lambda: _gated(residual=torch.zeros(M, N)), "bf16", _lib.EPI_GATE_RESIDUAL, TypeError,
     "residual must be bf16"),
    (lambda: _prob("fp8", a_scale=torch.ones(M - 1)), "fp8", _lib.EPI_NONE, ValueError,
     "a_scale must be"),
    (lambda: _prob("fp8", w_scale=torch.ones(N - 4)), "fp8", _lib.EPI_NONE, ValueError,
     "w_scale must be"),
    (lambda: _prob("fp8", w_scale=_bf16(N)), "fp8", _lib.EPI_NONE, TypeError, "w_scale must be"),
    (lambda: Problem(torch.zeros(M, K, dtype=torch.float8_e4m3fn),
                     torch.zeros(N, K, dtype=torch.float8_e4m3fn), _bf16(M, N)), "fp8",
     _lib.EPI_NONE, ValueError, "need a_scale and w_scale"),
    (lambda: _prob("mx", a_scale=torch.zeros(M, K // 64, dtype=torch.uint8)), "mx",
     _lib.EPI_NONE, ValueError, "a_scale must be contiguous"),
    (lambda: _prob("mx", w_scale=torch.zeros(N - 1, K // 32, dtype=torch.uint8)), "mx",
     _lib.EPI_NONE, ValueError, "w_scale must be contiguous"),
    (lambda: _prob("mx", w_scale=torch.zeros(K // 32, N, dtype=torch.uint8).T), "mx",
     _lib.EPI_NONE, ValueError, "w_scale must be contiguous"),
    (lambda: _prob("mx", a_scale=torch.zeros(M, K // 32)), "mx", _lib.EPI_NONE, TypeError,
     "a_scale must be uint8"),
])
def test_short_or_mistyped_epilogue_operands_are_refused(make, kind, epi, exc, msg):
    with pytest.raises(exc, match=msg):
        _run(make(), kind, epi)


def _tables(rows):
    return torch.zeros(rows, 128), torch.zeros(rows, 128)


def test_rope_rows_past_the_tables_are_refused():
    cos, sin = _tables(M + 10)
    qk = QkNormRope(0, 256, 256, cos, sin)
    with pytest.raises(ValueError, match=DEVICE_MSG):
        _run(_prob(rope_row0=10), qk=qk)
    with pytest.raises(ValueError, match="exceed the 310-row tables"):
        _run(_prob(rope_row0=11), qk=qk)
    with pytest.raises(ValueError, match="exceed"):
        _run(_prob(rope_row0=-1), qk=qk)
    c2, s2 = _tables(M + 10)
    with pytest.raises(ValueError, match="differ in shape"):
        _run(_prob(), qk=QkNormRope(0, 256, 256, c2, s2[:-1]))
    with pytest.raises(ValueError, match="norm weights"):
        _run(_prob(norm_q=_bf16(64)), qk=qk)
    with pytest.raises(ValueError, match="norm weights"):
        _run(_prob(norm_k=torch.ones(128)), qk=qk)


def test_the_c_abi_bounds_the_rope_rows_itself():
    """difflet_gemm_qk.rows: the library refuses a problem whose RoPE rows run past the tables
    before any device call (placeholder addresses, never dereferenced)."""
    lib = _lib.load()
    fake = 1 << 20  # 16-byte aligned, never read: the call fails in validation
    probs = (_lib.GemmProblem * 1)()
    p = probs[0]
    p.a, p.w, p.c = fake, fake, fake
    p.lda, p.ldw, p.ldc = K, K, N
    p.m, p.rows_per_batch, p.rope_row0 = M, M, 20
    qk = _lib.GemmQk(0, 256, 256, fake, fake, 0, 1e-6, M + 19)
    st = lib.difflet_rocm_gemm_bf16(1, probs, N, K, _lib.EPI_NONE, 0, None, 0, ctypes.byref(qk),
                                    None)
    assert st == _lib.EINVAL
    assert b"RoPE rows up to 320 of a 319-row table" in lib.difflet_rocm_last_error()


def test_problems_without_rows_are_dropped_before_any_check():
    """A grouped launch whose text part is empty (an empty prompt) runs its other problems; a
    launch with no rows at all returns at once (an empty tensor may have no address)."""
    empty = Problem(_bf16(0, K), _bf16(N, K), _bf16(0, N), gate=_bf16(1, N),
                    residual=_bf16(0, N))
    kernels.gemm_grouped([empty], epilogue=_lib.EPI_GATE_RESIDUAL)
    with pytest.raises(ValueError, match=DEVICE_MSG):
        kernels.gemm_grouped([empty, _gated()], epilogue=_lib.EPI_GATE_RESIDUAL)


def test_fp32_output_epilogue_checks():
    """EPI_F32: fp32 C from the bf16 GEMM only, 16-byte rows, no q/k norm."""
    f32 = Problem(_bf16(M, K), _bf16(N, K), torch.zeros(M, N))
    with pytest.raises(ValueError, match=DEVICE_MSG):
        _run(f32, "bf16", _lib.EPI_F32)
    with pytest.raises(ValueError, match="fp32 C"):
        _run(_prob(), "bf16", _lib.EPI_F32)  # bf16 C
    with pytest.raises(ValueError, match="fp32 C"):
        _run(Problem(_bf16(M, K), _bf16(N, K), torch.zeros(M, N + 2)[:, :N]), "bf16",
             _lib.EPI_F32)
    with pytest.raises(ValueError, match="bf16 GEMM"):
        _run(_prob("fp8"), "fp8", _lib.EPI_F32)
