"""Pins of the per-row e4m3 law (oracle/fp8.py), CPU only.

The law has no reference counterpart (the reference's only fp8 recipe is MXFP8); it is pinned
by its closed-form invariants and by torch's own float8 cast of the same fp32 products.
"""

import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle import mx as omx


def _rows(seed=0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((50, 384)) * np.exp(rng.standard_normal((50, 1)) * 5)).astype(np.float32)
    x[0] = 0.0
    x[1, 17] = -3e4
    return x


def test_codes_are_torchs_cast_of_the_scaled_row():
    x = _rows()
    q, s = ofp8.quantize_rowwise(x)
    amax = np.maximum(np.abs(x).max(axis=1), np.float32(2.0 ** -112)).astype(np.float32)
    inv = (np.float32(448.0) / amax).astype(np.float32)
    ref = torch.from_numpy(np.clip((x * inv[:, None]).astype(np.float32), -448, 448)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref)
    assert np.array_equal(s, (amax / np.float32(448.0)).astype(np.float32))


def test_row_maximum_is_the_largest_code_and_zero_rows_stay_zero():
    x = _rows(1)
    q, s = ofp8.quantize_rowwise(x)
    idx = np.abs(x).argmax(axis=1)
    for r in range(1, x.shape[0]):
        assert q[r, idx[r]] & 0x7F == 0x7E  # +-448
    assert np.all(q[0] == 0) and s[0] > 0


def test_dequantized_rows_are_within_half_an_e4m3_step():
    x = _rows(2)
    q, s = ofp8.quantize_rowwise(x)
    back = ofp8.dequantize_rowwise(q, s)
    scaled = np.abs(x) / s[:, None]
    # normal range: relative step 2^-3 (half = 2^-4); subnormal range: absolute 2^-10 * scale
    tol = np.maximum(scaled * 2.0 ** -4, 2.0 ** -10) * s[:, None] * (1 + 1e-6)
    assert np.all(np.abs(back - x) <= tol)


def test_fp8_linear_is_the_scaled_integer_product():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((9, 256)).astype(np.float32)
    w = (rng.standard_normal((20, 256)) * 0.05).astype(np.float32)
    b = rng.standard_normal(20).astype(np.float32)
    wq, ws = ofp8.quantize_rowwise(w)
    y = ofp8.fp8_linear(x, wq, ws, b)
    xq, xs = ofp8.quantize_rowwise(x)
    manual = (omx.e4m3_decode(xq).astype(np.float64) @ omx.e4m3_decode(wq).astype(np.float64).T
              ) * xs[:, None] * ws[None, :] + b
    assert np.allclose(y, manual, rtol=1e-5, atol=1e-5)
    exact = x @ w.T + b
    assert np.linalg.norm(y - exact) / np.linalg.norm(exact) < 0.06


def test_torch_twin_of_the_row_law_is_bit_exact():
    """fake_quantize_rowwise_torch / fp8_linear_torch (the threaded twins the block oracles
    use) equal the numpy law bit for bit: codes, scales and the linear's output."""
    import torch

    rng = np.random.default_rng(3)
    x = (rng.standard_normal((9, 256)) * np.exp2(rng.integers(-30, 30, size=(9, 1)))).astype(np.float32)
    x[4] = 0.0
    x[5, :3] = [448.0, -1e-30, 3e-39]
    q, s = ofp8.quantize_rowwise(x)
    tq, ts = ofp8.fake_quantize_rowwise_torch(torch.from_numpy(x))
    assert np.array_equal(tq.numpy(), omx.e4m3_decode(q))
    assert np.array_equal(ts.numpy().view(np.uint32), s.view(np.uint32))
    w = (rng.standard_normal((40, 256)) * 0.02).astype(np.float32)
    b = rng.standard_normal(40).astype(np.float32)
    wq, ws = ofp8.quantize_rowwise(w)
    want = ofp8.fp8_linear(x, wq, ws, b)
    got = ofp8.fp8_linear_torch(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b))
    assert np.allclose(got.numpy(), want, rtol=1e-6, atol=1e-6)
