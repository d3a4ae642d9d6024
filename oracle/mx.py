"""The MXFP8 block law of difflet/quant/mx.py restated in numpy integer arithmetic, plus an
fp32 -> float8_e4m3fn encoder. Test infrastructure only (see oracle/__init__.py).

Pins (tests/test_oracle_mx.py): the e4m3 encoder against torch's `.to(torch.float8_e4m3fn)`
on every fp32 rounding boundary of the format; `swizzle_perm` against an independent
reshape/transpose statement of the partition-x-byte layout described at difflet/quant/mx.py:17-27
and against the reference's own test assertions (tests/unit/quant/test_mx.py:74-83); the
scale law against its closed-form invariant (block max lands in [128, 256), mx.py:12-15).
"""

from __future__ import annotations

import numpy as np

BLOCK = 32          # difflet/quant/spec.py:39
LAYOUT_K = 128      # difflet/quant/spec.py:40
TILE_K = 512        # difflet/quant/mx.py:42
E4M3_MAX = 448.0    # difflet/quant/mx.py:41
E4M3_MAX_EXP = 7    # difflet/quant/mx.py:40
E8M0_BIAS = 127     # difflet/quant/mx.py:43


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> float8_e4m3fn codes (uint8), round to nearest even; inputs beyond +-448 (not
    produced by the quantizers, which clamp) saturate to +-448, NaN -> 0x7f | sign."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint32)
    a = u & np.uint32(0x7FFFFFFF)
    normal = ((a + np.uint32(0x7FFFF) + ((a >> 20) & 1)) >> 20) - np.uint32(120 << 3)
    sub = np.rint(a.view(np.float32) * np.float32(512.0)).astype(np.uint32)
    code = np.where(a < 0x3C800000, sub, normal)
    code = np.where(a >= 0x43E00000, np.uint32(0x7E), code)
    code = np.where(a > 0x7F800000, np.uint32(0x7F), code)
    return (code | sign).astype(np.uint8)


def _e4m3_table() -> np.ndarray:
    c = np.arange(256, dtype=np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8.0) * 2.0 ** (e - 7))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return (s * val).astype(np.float32)


_E4M3 = _e4m3_table()


def e4m3_decode(code: np.ndarray) -> np.ndarray:
    """float8_e4m3fn codes -> fp32 values (exact): sign * 2^(e-7) * (1 + m/8), subnormals
    m * 2^-9, code 0x7f / 0xff NaN."""
    return _E4M3[np.asarray(code, dtype=np.uint8)]


def tile_sizes(k: int) -> list[int]:
    """difflet/quant/mx.py:46-62: 512-wide tiles, then the whole remainder as one tile."""
    if k % LAYOUT_K:
        raise ValueError(f"K={k} must be a multiple of {LAYOUT_K} for the MX layout")
    tiles = [TILE_K] * (k // TILE_K)
    if k % TILE_K:
        tiles.append(k % TILE_K)
    return tiles


def swizzle_perm(k: int) -> np.ndarray:
    """difflet/quant/mx.py:65-76: perm[r * 4 + j] = k0 + j * (tile / 4) + r."""
    perm = []
    k0 = 0
    for tile in tile_sizes(k):
        sub = tile // 4
        for r in range(sub):
            for j in range(4):
                perm.append(k0 + j * sub + r)
        k0 += tile
    return np.asarray(perm, dtype=np.int64)


def block_scales(sw: np.ndarray) -> np.ndarray:
    """difflet/quant/mx.py:85-93: uint8 scale = clamp(max exponent field - 7, 0, 255) over each
    32 consecutive values of the swizzled fp32 rows."""
    e = (np.ascontiguousarray(sw, dtype=np.float32).view(np.uint32) >> 23) & 0xFF
    emax = e.reshape(*sw.shape[:-1], -1, BLOCK).max(axis=-1).astype(np.int64)
    return np.clip(emax - E4M3_MAX_EXP, 0, 255).astype(np.uint8)


def quantize_mx(t: np.ndarray, swizzled_out: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """difflet/quant/mx.py:96-108: [R, K] -> (e4m3 codes uint8 [R, K], E8M0 uint8 [R, K/32]).
    Codes in logical K order (the reference's storage) unless swizzled_out."""
    t = np.asarray(t, dtype=np.float32)
    k = t.shape[-1]
    perm = swizzle_perm(k)
    sw = t[..., perm]
    s = block_scales(sw)
    value = np.ldexp(np.float32(1.0), s.astype(np.int32) - E8M0_BIAS).astype(np.float32)
    scaled = (sw.reshape(*sw.shape[:-1], -1, BLOCK) / value[..., None]).astype(np.float32)
    q_sw = e4m3_encode(np.clip(scaled, -E4M3_MAX, E4M3_MAX).reshape(sw.shape))
    if swizzled_out:
        return q_sw, s
    q = np.empty_like(q_sw)
    q[..., perm] = q_sw
    return q, s


def dequantize_mx(q: np.ndarray, s: np.ndarray, swizzled_in: bool = False) -> np.ndarray:
    """difflet/quant/mx.py:111-120: fp32 [R, K] in logical order."""
    k = q.shape[-1]
    perm = swizzle_perm(k)
    qs = q if swizzled_in else q[..., perm]
    value = np.ldexp(np.float32(1.0), s.astype(np.int32) - E8M0_BIAS).astype(np.float32)
    sw = (e4m3_decode(qs).reshape(*q.shape[:-1], -1, BLOCK) * value[..., None]).reshape(q.shape)
    out = np.empty(q.shape, dtype=np.float32)
    out[..., perm] = sw
    return out


def fake_quantize_mx(t: np.ndarray) -> np.ndarray:
    return dequantize_mx(*quantize_mx(t))


def mx_linear(x: np.ndarray, wq: np.ndarray, ws: np.ndarray, bias=None) -> np.ndarray:
    """FakeQuantMXLinear.forward (difflet/quant/fake_linear.py:56-61) in fp32:
    mx(x) @ deq(W)^T + b (dequantized values are exact in fp32; the product is an fp32 matmul)."""
    import torch

    xq = torch.from_numpy(fake_quantize_mx(x.reshape(-1, x.shape[-1])))
    y = (xq @ torch.from_numpy(dequantize_mx(wq, ws)).T).numpy()
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return y.reshape(*x.shape[:-1], wq.shape[0]).astype(np.float32)


# ------------------------------------------------------------- torch twin for large blocks
def _e8m0_values_torch(s):
    """2^(s - 127) in fp32 for uint8 scales s (as int32), built from the bit pattern: exact,
    including s = 0 (the subnormal 2^-127)."""
    import torch

    bits = torch.where(s > 0, s << 23, torch.full_like(s, 0x400000))
    return bits.view(torch.float32)


def fake_quantize_mx_torch(t):
    """quantize_mx then dequantize_mx of a torch fp32 [..., K] tensor, in torch's threaded
    element-wise ops: the same block law step for step (swizzle, exponent-field maxima,
    IEEE fp32 divide, clamp, RNE e4m3 through torch's float8_e4m3fn cast, which is pinned equal
    to e4m3_encode on every rounding boundary). Pinned bit-exact against the numpy functions
    above (tests/test_oracle_mx.py); the block oracles use it for their large linears."""
    import torch

    t = t.to(torch.float32)
    k = t.shape[-1]
    perm = torch.from_numpy(swizzle_perm(k))
    sw = t.index_select(-1, perm).reshape(*t.shape[:-1], k // BLOCK, BLOCK).contiguous()
    e = (sw.view(torch.int32) >> 23) & 0xFF
    s = (e.amax(dim=-1) - E4M3_MAX_EXP).clamp(0, 255)
    value = _e8m0_values_torch(s.to(torch.int32))[..., None]
    q = (sw / value).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    deq = (q.to(torch.float32) * value).reshape(*t.shape[:-1], k)
    out = torch.empty_like(deq)
    out.index_copy_(-1, perm, deq)
    return out

