"""Pins of the oracle's MXFP8 law (oracle/mx.py) and e4m3 encoder, CPU only.

Each check compares against something other than the oracle's own formula: torch's float8 cast
(a library routine), an independent reshape/transpose statement of the swizzle described at
difflet/quant/mx.py:17-27, a brute-force nearest-value search over the 256 e4m3 codes, the
reference tests' own assertions (tests/unit/quant/test_mx.py:62-83), and the law's closed-form
invariant (the block maximum lands in [128, 256), difflet/quant/mx.py:12-15).
"""

import math

import numpy as np
import pytest
import torch

from oracle import mx as omx


def torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encoder_matches_torch_on_every_rounding_boundary():
    """All representable values, every tie between neighbours, and one fp32 ulp either side."""
    reps = np.unique(np.abs(omx.e4m3_decode(np.arange(256, dtype=np.uint8))))
    reps = reps[np.isfinite(reps)].astype(np.float64)
    mids = (reps[:-1] + reps[1:]) / 2
    pts = np.concatenate([reps, mids]).astype(np.float32)
    bits = pts.view(np.uint32)
    around = np.concatenate([bits - 1, bits, bits + 1]).view(np.float32)
    around = around[np.abs(around) <= 448]
    x = np.concatenate([around, -around, [0.0, -0.0]]).astype(np.float32)
    assert np.array_equal(omx.e4m3_encode(x), torch_e4m3(x))


def test_e4m3_encoder_matches_torch_on_a_strided_sweep_of_fp32():
    """Every 97th fp32 bit pattern from 0 up to 448 (about 11M values), both signs."""
    top = np.float32(448.0).view(np.uint32)
    bits = np.arange(0, int(top) + 1, 97, dtype=np.uint32)
    x = bits.view(np.float32)
    x = np.concatenate([x, -x])
    assert np.array_equal(omx.e4m3_encode(x), torch_e4m3(x))


def test_e4m3_decode_round_trips_every_finite_code():
    codes = np.arange(256, dtype=np.uint8)
    vals = omx.e4m3_decode(codes)
    finite = np.isfinite(vals)
    assert np.array_equal(omx.e4m3_encode(vals[finite]), codes[finite])
    assert np.array_equal(torch_e4m3(vals[finite]), codes[finite])


def _perm_by_reshape(k):
    """The partition x byte layout read straight from its description: each K tile (512, or the
    whole remainder) spread over tile/4 partitions, the tile's four quarters as the four bytes
    of each partition; blocks are 8 partitions x 4 bytes."""
    out, k0 = [], 0
    while k0 < k:
        t = min(512, k - k0) if (k - k0) >= 512 else k - k0
        quarters = np.arange(k0, k0 + t).reshape(4, t // 4)  # [byte j, partition p]
        out.append(quarters.T.reshape(-1))                    # partition-major, then byte
        k0 += t
    return np.concatenate(out)


@pytest.mark.parametrize("k", [128, 256, 384, 512, 768, 896, 1536, 3072, 3456, 13824, 15360])
def test_swizzle_perm_is_the_partition_byte_layout(k):
    perm = omx.swizzle_perm(k)
    assert sorted(perm.tolist()) == list(range(k))
    assert np.array_equal(perm, _perm_by_reshape(k))


def test_k_must_be_a_multiple_of_128():
    with pytest.raises(ValueError):
        omx.swizzle_perm(96)


def test_one_swizzled_block_scales_alone():
    """tests/unit/quant/test_mx.py:74-83."""
    k = 512
    perm = omx.swizzle_perm(k)
    x = np.zeros((1, k), np.float32)
    x[0, perm[:32]] = 1.0
    x[0, perm[0]] = 100.0
    q, s = omx.quantize_mx(x)
    assert (s[0] != s[0, 1]).sum() == 1
    assert s[0, 0] > s[0, 1]


def test_round_trip_and_outlier_isolation():
    """tests/unit/quant/test_mx.py:62-71."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4, 3072)).astype(np.float32)
    x[0, 7] = 1000.0
    back = omx.fake_quantize_mx(x)
    assert np.linalg.norm(back - x) / np.linalg.norm(x) < 0.05
    far = slice(2048, 2048 + 32)
    assert (np.abs(back[1, far] - x[1, far]) / np.abs(x[1, far])).max() < 0.07
    assert (back[0] != 0).mean() > 0.9


def test_block_maximum_lands_in_128_256():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 1024)) * np.exp(rng.standard_normal((64, 1)) * 4)).astype(np.float32)
    perm = omx.swizzle_perm(1024)
    s = omx.quantize_mx(x)[1].astype(np.int64)
    blocks = np.abs(x[:, perm]).reshape(64, -1, 32).max(axis=-1).astype(np.float64)
    scaled = blocks / np.exp2(s - 127.0)
    assert np.all((scaled >= 128) & (scaled < 256))


def _nearest_e4m3(v):
    """Brute force: the e4m3 code whose value is nearest, ties to the even code."""
    codes = np.arange(256, dtype=np.uint8)
    vals = omx.e4m3_decode(codes).astype(np.float64)
    ok = np.isfinite(vals)
    best = None
    for c, val in zip(codes[ok], vals[ok]):
        d = abs(val - v)
        if best is None or d < best[0] - 1e-300 or (d == best[0] and (c & 1) == 0 and (best[1] & 1)):
            best = (d, int(c))
    return best[1]


def test_quantize_mx_matches_brute_force_on_tiny_blocks():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((2, 128)) * np.array([[1e-3], [30.0]])).astype(np.float32)
    x[0, 3] = 0.0
    q, s = omx.quantize_mx(x)
    perm = omx.swizzle_perm(128)
    for r in range(2):
        for b in range(4):
            idx = perm[b * 32:(b + 1) * 32]
            vals = x[r, idx].astype(np.float64)
            emax = max((math.frexp(abs(v))[1] + 126) if v != 0 else 0 for v in vals)
            su = min(max(emax - 7, 0), 255)
            assert s[r, b] == su
            for kk, v in zip(idx, vals):
                scaled = min(max(v / 2.0 ** (su - 127), -448.0), 448.0)
                code = _nearest_e4m3(scaled)
                got = int(q[r, kk])
                # +-0: the encoder keeps the sign bit, the nearest search may pick either zero
                if omx.e4m3_decode(np.uint8(code)) == 0:
                    assert omx.e4m3_decode(np.uint8(got)) == 0
                else:
                    assert got == code


def test_tiles_quantize_independently():
    """Block membership is local to 512-wide tiles: quantizing [R, 1024] equals quantizing its
    two 512-wide halves (the basis of quantizing a row-parallel shard on its own)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 1024)).astype(np.float32)
    q, s = omx.quantize_mx(x)
    q0, s0 = omx.quantize_mx(x[:, :512])
    q1, s1 = omx.quantize_mx(x[:, 512:])
    assert np.array_equal(q, np.concatenate([q0, q1], axis=1))
    assert np.array_equal(s, np.concatenate([s0, s1], axis=1))


def test_swizzled_storage_is_the_permuted_logical_storage():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 896)).astype(np.float32)
    ql, sl = omx.quantize_mx(x)
    qs, ss = omx.quantize_mx(x, swizzled_out=True)
    assert np.array_equal(ss, sl)
    assert np.array_equal(qs, ql[:, omx.swizzle_perm(896)])
    assert np.allclose(omx.dequantize_mx(qs, ss, swizzled_in=True), omx.dequantize_mx(ql, sl))


def test_mx_linear_is_the_block_law_in_fp32():
    """FakeQuantMXLinear's law (tests/unit/quant/test_fake_linear.py:21-35): y = deq(q(x)) @
    deq(q(W))^T + b, and close to the unquantized product."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((7, 256)).astype(np.float32)
    w = (rng.standard_normal((33, 256)) * 0.05).astype(np.float32)
    b = rng.standard_normal(33).astype(np.float32)
    wq, ws = omx.quantize_mx(w)
    y = omx.mx_linear(x, wq, ws, b)
    manual = omx.fake_quantize_mx(x) @ omx.dequantize_mx(wq, ws).T + b
    assert np.allclose(y, manual, rtol=1e-5, atol=1e-5)
    exact = x @ w.T + b
    assert np.linalg.norm(y - exact) / np.linalg.norm(exact) < 0.05


@pytest.mark.parametrize("k", [128, 384, 896, 3072])
def test_torch_twin_of_the_block_law_is_bit_exact(k):
    """fake_quantize_mx_torch (the threaded twin the block oracles use) equals
    dequantize_mx(quantize_mx(.)) bit for bit, over wide-range values, zeros, subnormals,
    exact powers of two and e4m3 midpoints scaled by every block exponent."""
    import torch

    rng = np.random.default_rng(k)
    rows = [rng.standard_normal(k) * np.exp2(rng.integers(-40, 40, size=k)),
            np.zeros(k), rng.standard_normal(k) * 1e-40,
            np.exp2(rng.integers(-126, 127, size=k)) * rng.choice([-1, 1], size=k)]
    mids = omx.e4m3_decode(np.arange(0x7e, dtype=np.uint8))
    mids = ((mids[1:] + mids[:-1]) / 2).astype(np.float32)
    rows.append(np.resize(mids, k) * np.exp2(rng.integers(-20, 20, size=k)))
    x = np.stack(rows).astype(np.float32)
    want = omx.dequantize_mx(*omx.quantize_mx(x))
    got = omx.fake_quantize_mx_torch(torch.from_numpy(x)).numpy()
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32))
