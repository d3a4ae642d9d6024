"""The per-row e4m3 law of the per-channel (weights) x per-token (activations) fp8 linear.
Test infrastructure only (see oracle/__init__.py).

There is no reference counterpart: the reference's only fp8 recipe is MXFP8
(difflet/quant/spec.py:22-33). The law is this build's and is fixed in include/difflet_rocm.h
(difflet_rocm_quantize_fp8_rowwise): amax = max |x|, a = max(amax, 2^-112), scale = a / 448,
inv = 448 / a (IEEE fp32 divisions), q = e4m3_rne(clamp(x * inv, -448, 448)).

Pins (tests/test_oracle_fp8.py): the e4m3 encoder is pinned in oracle/mx.py; the row law
against its closed-form invariants (the row's amax encodes to +-448 = code 0x7e, dequantized
rows are within e4m3's half-ulp of the input, a zero row gives zero codes) and against torch's
own float8 cast of the same fp32 products.
"""

from __future__ import annotations

import numpy as np

from oracle.mx import e4m3_decode, e4m3_encode

E4M3_MAX = np.float32(448.0)
TINY = np.float32(2.0 ** -112)  # 448 / TINY is finite in fp32


def quantize_rowwise(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[R, K] -> (codes uint8 [R, K], fp32 scales [R])."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=-1)
    a = np.maximum(amax, TINY).astype(np.float32)
    scale = (a / E4M3_MAX).astype(np.float32)
    inv = (E4M3_MAX / a).astype(np.float32)
    prod = (x * inv[..., None]).astype(np.float32)
    q = e4m3_encode(np.clip(prod, -E4M3_MAX, E4M3_MAX))
    return q, scale


def dequantize_rowwise(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    return (e4m3_decode(q) * scale[..., None]).astype(np.float32)


def fp8_linear(x: np.ndarray, wq: np.ndarray, ws: np.ndarray, bias=None) -> np.ndarray:
    """y = (q_x q_w^T) * s_x[m] * s_w[n] + b with an fp32 product: what the fp8 GEMM computes.
    Products of two e4m3 values are exact in fp32; the sum is an fp32 matmul."""
    import torch

    x2 = np.asarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    xq, xs = quantize_rowwise(x2)
    acc = torch.from_numpy(e4m3_decode(xq)) @ torch.from_numpy(e4m3_decode(wq)).T
    y = (acc * torch.from_numpy(xs)[:, None] * torch.from_numpy(ws)[None, :]).numpy()
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return y.reshape(*x.shape[:-1], wq.shape[0]).astype(np.float32)


def fake_quantize_rowwise_torch(x):
    """quantize_rowwise then dequantize_rowwise in torch's threaded element-wise ops, the same
    law step for step (e4m3 through torch's float8_e4m3fn cast, pinned equal to e4m3_encode).
    Returns (dequantized codes [R, K] fp32 without the scale, scales [R]); pinned bit-exact
    against the numpy functions (tests/test_oracle_fp8.py)."""
    import torch

    x = x.to(torch.float32)
    amax = x.abs().amax(dim=-1)
    a = torch.clamp_min(amax, float(TINY))
    scale = a / float(E4M3_MAX)
    inv = float(E4M3_MAX) / a
    q = (x * inv[..., None]).clamp(-float(E4M3_MAX), float(E4M3_MAX)).to(torch.float8_e4m3fn)
    return q.to(torch.float32), scale


def fp8_linear_torch(x, w, bias=None):
    """fp8_linear on torch fp32 operands, quantizing both rows-wise here: what the per-token x
    per-channel fp8 GEMM computes for activations x [..., K] and weights w [N, K]."""
    x2 = x.reshape(-1, x.shape[-1])
    xq, xs = fake_quantize_rowwise_torch(x2)
    wq, ws = fake_quantize_rowwise_torch(w)
    y = (xq @ wq.T) * xs[:, None] * ws[None, :]
    if bias is not None:
        y = y + bias
    return y.reshape(*x.shape[:-1], w.shape[0])

