"""torch-facing wrappers of the C ABI: validate tensors, pick strides, call libdifflet_rocm.

Every function here runs a HIP kernel on the tensors' device, on torch's current stream. There
is no CPU or eager-torch path: a CPU tensor, an unsupported dtype or a missing library raises.
Outputs are allocated with torch (the library never allocates).
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from difflet_amd import _lib
from difflet_amd._lib import GemmProblem, check

_DT = {
    torch.float32: _lib.F32,
    torch.bfloat16: _lib.BF16,
    torch.float16: _lib.F16,
    torch.uint8: _lib.U8,
    torch.bool: _lib.BOOL,
    torch.int32: _lib.I32,
    torch.float8_e4m3fn: _lib.U8,
}
FLOAT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def lib():
    return _lib.load()


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"dtype {t.dtype} is not supported by the rocm kernels") from None


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _on_gpu(*ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"rocm kernels take device tensors, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def _arr(vals: Sequence[int]):
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


def _rows2d(t: torch.Tensor, name: str) -> torch.Tensor:
    """A [rows, cols] view with contiguous rows (copies only if the innermost dim is strided)."""
    if t.dim() < 1:
        raise ValueError(f"{name}: needs at least one dimension")
    t2 = t.reshape(-1, t.shape[-1]) if t.dim() != 2 else t
    if t2.stride(-1) != 1:
        t2 = t2.contiguous()
    return t2


# ------------------------------------------------------------------------------- attention
def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float,
              causal: bool = False, attention_mask: torch.Tensor | None = None,
              bound_min: torch.Tensor | None = None, bound_max: torch.Tensor | None = None,
              out: torch.Tensor | None = None,
              workspace: torch.Tensor | None | str = "shared") -> torch.Tensor:
    """softmax(q k^T scale [+ mask]) v on [B, H, S, D] (or [B*H, S, D]) tensors.

    workspace: "shared" (the workspace of the current stream, see attention_workspace), a
    zero-filled uint8 tensor of attention_workspace_bytes(), or None (every query tile runs
    whole on one workgroup)."""
    dev = _on_gpu(q, k, v)
    folded = q.dim() == 3
    scores_shape = tuple(q.shape[:-1]) + (k.shape[-2],)
    if folded:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("attention takes [B, H, S, D] or [B*H, S, D] tensors")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v dtypes differ: {q.dtype}, {k.dtype}, {v.dtype}")
    b, h, sq, d = q.shape
    sk = k.shape[2]
    if k.shape != (b, h, sk, d) or v.shape != (b, h, sk, d):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    if out is None:
        out = torch.empty((b, h, sq, d), dtype=v.dtype, device=dev)
        o = out
        out = out[0] if folded else out
    else:
        o = out.unsqueeze(0) if folded else out
    mask_ptr, mask_dt, mask_strides = None, 0, None
    keep = []
    if attention_mask is not None:
        if bound_min is not None or bound_max is not None:
            raise ValueError("attention_mask and bounds are mutually exclusive")
        m = attention_mask.to(dev)
        if m.dtype == torch.bool:
            m, mask_dt = m.view(torch.uint8), _lib.BOOL
        else:
            if m.dtype not in FLOAT_DTYPES:
                m = m.to(q.dtype)
            mask_dt = _dt(m)
        m = torch.broadcast_to(m, scores_shape)  # a view: broadcast dims get stride 0
        m = m.unsqueeze(0) if folded else m
        keep.append(m)
        mask_ptr = ctypes.c_void_p(m.data_ptr())
        mask_strides = _arr(m.stride())
    bmin_ptr = bmax_ptr = bstr = None
    if bound_min is not None or bound_max is not None:
        if bound_min is None or bound_max is None:
            raise ValueError("bound_min and bound_max must both be provided")
        # bounds broadcast against the scores with a trailing key dim of 1
        def _as_bhq(t):
            t = torch.broadcast_to(t.to(device=dev, dtype=torch.int32), scores_shape[:-1] + (1,))
            t = t[..., 0]
            return (t.unsqueeze(0) if folded else t).contiguous()
        bmn, bmx = _as_bhq(bound_min), _as_bhq(bound_max)
        keep += [bmn, bmx]
        bmin_ptr, bmax_ptr = _ptr(bmn), _ptr(bmx)
        bstr = _arr(bmn.stride())
    if isinstance(workspace, str):
        if workspace != "shared":
            raise ValueError(f"workspace must be 'shared', a tensor or None, not {workspace!r}")
        workspace = attention_workspace(dev)
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel())
    st = lib().difflet_rocm_attention(
        _ptr(q), _ptr(k), _ptr(v), _ptr(o), _dt(q), b, h, sq, sk, d,
        _arr(q.stride()[:3]), _arr(k.stride()[:3]), _arr(v.stride()[:3]), _arr(o.stride()[:3]),
        float(scale), int(bool(causal)), mask_ptr, mask_dt, mask_strides, bmin_ptr, bmax_ptr,
        bstr, ws_ptr, ws_bytes, _stream(dev))
    check(st, "attention")
    return out


# ------------------------------------------------------------------------------------ GEMM
class Problem:
    """One problem of a grouped GEMM: C = epilogue(A W^T + bias)."""

    __slots__ = ("a", "w", "c", "bias", "gate", "residual", "a_scale", "w_scale",
                 "rows_per_batch", "norm_q", "norm_k", "rope_row0", "c_scale")

    def __init__(self, a, w, c, bias=None, gate=None, residual=None, a_scale=None,
                 w_scale=None, rows_per_batch=None, norm_q=None, norm_k=None, rope_row0=0,
                 c_scale=None):
        self.a, self.w, self.c = a, w, c
        self.bias, self.gate, self.residual = bias, gate, residual
        self.a_scale, self.w_scale = a_scale, w_scale
        self.rows_per_batch = rows_per_batch
        # fused q/k norm (gemm_grouped(..., qk=QkNormRope)): this problem's [128] bf16 RMSNorm
        # weights and the RoPE table row of its row 0
        self.norm_q, self.norm_k, self.rope_row0 = norm_q, norm_k, rope_row0
        # EPI_GELU_MX: c holds e4m3 codes and c_scale the E8M0 scales [m, n / 32]
        self.c_scale = c_scale


class QkNormRope:
    """Fused q/k RMSNorm + RoPE epilogue of a GEMM whose output holds 128-column q and k heads
    in columns [q_col, q_col + cols) and [k_col, k_col + cols) (multiples of 256; None skips
    one): the GEMM followed by qk_norm_rope(do_norm=True), up to fp32 summation order. cos / sin
    are fp32 [rows, 128] tables indexed by each problem's rope_row0 + row."""

    __slots__ = ("q_col", "k_col", "cols", "cos", "sin", "law", "eps")

    def __init__(self, q_col, k_col, cols, cos, sin, *, law=0, eps=1e-6):
        self.q_col, self.k_col, self.cols = q_col, k_col, cols
        self.cos, self.sin, self.law, self.eps = cos, sin, law, eps


_GEMM_FN = {"bf16": "difflet_rocm_gemm_bf16", "fp8": "difflet_rocm_gemm_fp8_rowwise",
            "mx": "difflet_rocm_gemm_mxfp8"}


_WORKSPACE: dict[tuple[int, int], torch.Tensor] = {}
_ATT_WORKSPACE: dict[tuple[int, int], torch.Tensor] = {}


def attention_workspace(dev: torch.device) -> torch.Tensor:
    """The attention workspace (split schedule) of the device's current stream, zero-filled
    once on first use. Launches on one stream run in order, so they can share it; each stream
    gets its own, since launches on different streams may overlap."""
    i = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (i, torch.cuda.current_stream(torch.device("cuda", i)).cuda_stream)
    ws = _ATT_WORKSPACE.get(key)
    if ws is None:
        with torch.cuda.device(i):
            nbytes = int(lib().difflet_rocm_attention_workspace_bytes())
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=torch.device("cuda", i))
        _ATT_WORKSPACE[key] = ws
    return ws


def gemm_workspace(dev: torch.device) -> torch.Tensor:
    """The split-GEMM workspace of the device's current stream, zero-filled once on first use
    (every launch leaves its counters at zero). Launches on one stream run in order, so they can
    share it; each stream gets its own, since launches on different streams may overlap."""
    i = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (i, torch.cuda.current_stream(torch.device("cuda", i)).cuda_stream)
    ws = _WORKSPACE.get(key)
    if ws is None:
        with torch.cuda.device(i):
            nbytes = int(lib().difflet_rocm_gemm_workspace_bytes())
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=torch.device("cuda", i))
        _WORKSPACE[key] = ws
    return ws


def _check_epilogue_operands(p: Problem, i: int, kind: str, n: int, k: int,
                             epilogue: int) -> None:
    """Every vector the GEMM kernel reads beside A and W, checked against what it reads: the
    kernel indexes bias[n], gate[row, n], residual[m, n], a_scale[m] and w_scale[n] (fp8), and
    the E8M0 rows a_scale[m, :k/32] / w_scale[n, :k/32] (MXFP8) without bounds checks of its
    own, so a short or mistyped tensor is refused here."""
    m = p.a.shape[0]

    def vec(t, what, dtype, length):
        if t.dtype != dtype:
            raise TypeError(f"problem {i}: {what} must be {dtype}, got {t.dtype}")
        if t.dim() != 1 or t.stride(0) != 1 or t.shape[0] < length:
            raise ValueError(f"problem {i}: {what} must be a contiguous vector of at least "
                             f"{length} values, got {tuple(t.shape)}")

    if p.bias is not None:
        vec(p.bias, "bias", torch.bfloat16, n)
    if epilogue == _lib.EPI_GATE_RESIDUAL:
        if p.gate is None or p.residual is None:
            raise ValueError(f"problem {i}: the gate/residual epilogue needs gate and residual")
        rpb = p.rows_per_batch or max(m, 1)
        batches = max(1, -(-m // rpb))
        g = p.gate if p.gate.dim() == 2 else p.gate.reshape(1, -1)
        if g.dtype != torch.bfloat16:
            raise TypeError(f"problem {i}: gate must be bf16, got {g.dtype}")
        if g.dim() != 2 or g.stride(-1) != 1 or g.shape[1] < n or g.shape[0] < batches:
            raise ValueError(f"problem {i}: gate must hold {batches} row(s) of at least {n} "
                             f"contiguous values, got {tuple(p.gate.shape)}")
        r = p.residual
        if r.dtype != torch.bfloat16:
            raise TypeError(f"problem {i}: residual must be bf16, got {r.dtype}")
        if r.dim() != 2 or r.stride(1) != 1 or r.shape[0] < m or r.shape[1] < n:
            raise ValueError(f"problem {i}: residual must be [>= {m}, >= {n}] with contiguous "
                             f"rows, got {tuple(r.shape)}")
    if kind == "fp8":
        if p.a_scale is None or p.w_scale is None:
            raise ValueError(f"problem {i}: fp8 GEMMs need a_scale and w_scale")
        vec(p.a_scale, "a_scale", torch.float32, m)
        vec(p.w_scale, "w_scale", torch.float32, n)
    elif kind == "mx":
        if p.a_scale is None or p.w_scale is None:
            raise ValueError(f"problem {i}: MXFP8 GEMMs need a_scale and w_scale")
        for t, what, rows in ((p.a_scale, "a_scale", m), (p.w_scale, "w_scale", n)):
            if t.dtype != torch.uint8:
                raise TypeError(f"problem {i}: {what} must be uint8 E8M0, got {t.dtype}")
            if t.dim() != 2 or tuple(t.shape) != (rows, k // 32) or not t.is_contiguous():
                raise ValueError(f"problem {i}: {what} must be contiguous [{rows}, {k // 32}], "
                                 f"got {tuple(t.shape)}")


def _check_qk(qk: QkNormRope, problems: Sequence[Problem]) -> None:
    """The fused q/k epilogue reads norm_q / norm_k [128] and the RoPE tables at rows
    rope_row0 .. rope_row0 + m - 1 of every problem."""
    for t in (qk.cos, qk.sin):
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != 128 or not t.is_contiguous():
            raise ValueError("RoPE tables are contiguous fp32 [rows, 128]")
    if qk.cos.shape != qk.sin.shape:
        raise ValueError("RoPE cos and sin tables differ in shape")
    rows = qk.cos.shape[0]
    for i, p in enumerate(problems):
        for t in (p.norm_q, p.norm_k):
            if t is not None and (t.dtype != torch.bfloat16 or t.numel() != 128
                                  or not t.is_contiguous()):
                raise ValueError("q/k norm weights are contiguous [128] bf16")
        lo, hi = int(p.rope_row0), int(p.rope_row0) + p.a.shape[0]
        if lo < 0 or hi > rows:
            raise ValueError(f"problem {i}: RoPE rows [{lo}, {hi}) exceed the {rows}-row tables")


def gemm_grouped(problems: Sequence[Problem], *, kind: str = "bf16",
                 epilogue: int = _lib.EPI_NONE, act_col_start: int = 0,
                 workspace: torch.Tensor | None | str = None,
                 qk: QkNormRope | None = None) -> None:
    """Runs up to 4 GEMMs sharing N, K and the epilogue in one launch (writes each p.c).
    workspace: None (every tile whole on one workgroup, the default), "shared" (the current
    stream's, see gemm_workspace) or a zero-filled uint8 tensor of
    difflet_rocm_gemm_workspace_bytes() bytes, which lets a launch whose last wave of tiles
    would be poorly filled cut those tiles along K over the XCDs when that takes a quarter and
    at least 24 K stages off its time (Qwen-Image's 336-tile projections, Wan's bf16 text k/v
    projection; FLUX's launches stay whole)."""
    # a problem without rows has nothing to compute (and an empty tensor may have no address)
    problems = [p for p in problems if p.a.shape[0] > 0]
    if not problems:
        return
    n, k = problems[0].w.shape[0], problems[0].w.shape[1]
    arr = (GemmProblem * len(problems))()
    for i, p in enumerate(problems):
        for t in (p.a, p.w, p.c):
            if t.dim() != 2 or t.stride(1) != 1:
                raise ValueError("GEMM operands must be 2-D with contiguous rows")
        if p.w.shape != (n, k) or p.a.shape[1] != k or p.c.shape != (p.a.shape[0], n):
            raise ValueError(f"GEMM shapes: a {tuple(p.a.shape)} w {tuple(p.w.shape)} "
                             f"c {tuple(p.c.shape)}")
        if kind == "bf16" and (p.a.dtype != torch.bfloat16 or p.w.dtype != torch.bfloat16):
            raise TypeError("bf16 GEMM takes bf16 operands")
        if kind != "bf16" and (p.a.element_size() != 1 or p.w.element_size() != 1):
            raise TypeError("fp8 GEMMs take e4m3 codes (uint8 or float8_e4m3fn)")
        if epilogue == _lib.EPI_GELU_MX:
            if kind != "mx":
                raise ValueError("the GELU -> MXFP8 epilogue runs on the MXFP8 GEMM only")
            cs = p.c_scale
            if p.c.element_size() != 1 or cs is None or cs.dtype != torch.uint8 or \
                    cs.dim() != 2 or cs.stride(1) != 1 or cs.shape[0] != p.a.shape[0] or \
                    cs.shape[1] < n // 32 or n % 32 or p.c.stride(0) % 8:
                raise ValueError("the GELU -> MXFP8 epilogue writes e4m3 codes [m, n] (row "
                                 "stride a multiple of 8) and uint8 scales [m, n / 32]; n % 32 "
                                 "== 0")
        elif epilogue == _lib.EPI_F32:
            if kind != "bf16" or qk is not None:
                raise ValueError("the fp32-output epilogue runs on the bf16 GEMM without the "
                                 "q/k norm")
            if p.c.dtype != torch.float32 or p.c.stride(0) % 4 or p.c.data_ptr() % 16:
                raise ValueError("the fp32-output epilogue writes fp32 C (row stride a multiple "
                                 "of 4, 16-byte aligned)")
        elif p.c.dtype != torch.bfloat16:
            raise TypeError("GEMM output is bf16")
        _check_epilogue_operands(p, i, kind, n, k, epilogue)
    if qk is not None:
        _check_qk(qk, problems)
    dev = _on_gpu(*[t for p in problems for t in (p.a, p.w, p.c, p.bias, p.gate, p.residual,
                                                  p.a_scale, p.w_scale)])
    for i, p in enumerate(problems):
        q = arr[i]
        q.a, q.lda = p.a.data_ptr(), p.a.stride(0)
        q.w, q.ldw = p.w.data_ptr(), p.w.stride(0)
        q.c, q.ldc = p.c.data_ptr(), p.c.stride(0)
        q.bias = p.bias.data_ptr() if p.bias is not None else None
        if p.gate is not None:
            g = p.gate if p.gate.dim() == 2 else p.gate.reshape(1, -1)
            q.gate, q.gate_stride = g.data_ptr(), (g.stride(0) if g.shape[0] > 1 else 0)
        if p.residual is not None:
            q.residual, q.ldr = p.residual.data_ptr(), p.residual.stride(0)
        q.a_scale = p.a_scale.data_ptr() if p.a_scale is not None else None
        q.w_scale = p.w_scale.data_ptr() if p.w_scale is not None else None
        q.m = p.a.shape[0]
        q.rows_per_batch = p.rows_per_batch or p.a.shape[0]
        if p.c_scale is not None and epilogue == _lib.EPI_GELU_MX:
            q.c_scale, q.ld_c_scale = p.c_scale.data_ptr(), p.c_scale.stride(0)
        if qk is not None:
            q.norm_q = p.norm_q.data_ptr() if p.norm_q is not None else None
            q.norm_k = p.norm_k.data_ptr() if p.norm_k is not None else None
            q.rope_row0 = int(p.rope_row0)
    if isinstance(workspace, str):
        if workspace != "shared":
            raise ValueError(f"workspace must be 'shared', a tensor or None, got {workspace!r}")
        workspace = gemm_workspace(dev)
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(),
                                                           workspace.numel())
    qk_arg = None
    if qk is not None:
        rows = qk.cos.shape[0]
        qk_arg = ctypes.byref(_lib.GemmQk(-1 if qk.q_col is None else qk.q_col,
                                          -1 if qk.k_col is None else qk.k_col, qk.cols,
                                          qk.cos.data_ptr(), qk.sin.data_ptr(), int(qk.law),
                                          float(qk.eps), rows))
    fn = getattr(lib(), _GEMM_FN[kind])
    check(fn(len(problems), arr, n, k, int(epilogue), int(act_col_start), ws_ptr, ws_bytes,
             qk_arg, _stream(dev)), f"gemm_{kind}")


def linear(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None, *,
           epilogue: int = _lib.EPI_NONE, gate: torch.Tensor | None = None,
           residual: torch.Tensor | None = None, act_col_start: int = 0,
           rows_per_batch: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 ``x W^T + b`` over the last dim of x, with an optional fused epilogue."""
    x2 = _rows2d(x, "linear")
    n = w.shape[0]
    c = out if out is not None else torch.empty((x2.shape[0], n), dtype=torch.bfloat16,
                                                device=x.device)
    res2 = _rows2d(residual, "residual") if residual is not None else None
    gemm_grouped([Problem(x2, w, c, bias, gate, res2, rows_per_batch=rows_per_batch)],
                 kind="bf16", epilogue=epilogue, act_col_start=act_col_start)
    return c.reshape(*x.shape[:-1], n) if out is None else c


# ------------------------------------------------------------------------------- quantizers
def quantize_fp8_rowwise(x: torch.Tensor, *, gelu_from: int | None = None
                         ) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row e4m3 codes (float8_e4m3fn [rows, K]) and fp32 scales [rows]. gelu_from (bf16 x,
    a multiple of 8): columns from there on are quantized as bf16(gelu_tanh(x)), the MLP
    activation applied where its pre-activation is quantized."""
    dev = _on_gpu(x)
    x2 = _rows2d(x, "quantize_fp8_rowwise")
    rows, cols = x2.shape
    q = torch.empty((rows, cols), dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty((rows,), dtype=torch.float32, device=dev)
    if gelu_from is None:
        check(lib().difflet_rocm_quantize_fp8_rowwise(_ptr(x2), _dt(x2), rows, cols,
                                                      x2.stride(0), _ptr(q), cols, _ptr(s),
                                                      _stream(dev)), "quantize_fp8_rowwise")
    else:
        check(lib().difflet_rocm_quantize_fp8_rowwise_gelu(_ptr(x2), _dt(x2), rows, cols,
                                                           x2.stride(0), _ptr(q), cols, _ptr(s),
                                                           int(gelu_from), _stream(dev)),
              "quantize_fp8_rowwise_gelu")
    return q, s


def quantize_mxfp8(x: torch.Tensor, *, swizzled: bool = False
                   ) -> tuple[torch.Tensor, torch.Tensor]:
    """MXFP8 codes (float8_e4m3fn [rows, K], logical or swizzle order) and uint8 E8M0 scales
    [rows, K/32] in block order."""
    dev = _on_gpu(x)
    x2 = _rows2d(x, "quantize_mxfp8")
    rows, cols = x2.shape
    q = torch.empty((rows, cols), dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty((rows, cols // 32), dtype=torch.uint8, device=dev)
    check(lib().difflet_rocm_quantize_mxfp8(_ptr(x2), _dt(x2), rows, cols, x2.stride(0), _ptr(q),
                                            cols, _ptr(s), cols // 32, int(swizzled),
                                            _stream(dev)),
          "quantize_mxfp8")
    return q, s


# ---------------------------------------------------------------------------- norms, rope
def layernorm_modulate(x: torch.Tensor, mul: torch.Tensor | None, add: torch.Tensor | None, *,
                       eps: float, one_plus: bool = True, out_dtype: torch.dtype | None = None,
                       rows_per_batch: int | None = None, split: int = 0,
                       mul2: torch.Tensor | None = None, add2: torch.Tensor | None = None,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """LN(x) * (1 + mul) + add (one_plus) or LN(x) * mul + add, over the last dim.

    mul / add: [dim] or [batches, dim], broadcast over the rows of each batch element. With
    split > 0, rows >= split take mul2 / add2 instead (two segments in one launch)."""
    dev = _on_gpu(x)
    x2 = _rows2d(x, "layernorm")
    rows, dim = x2.shape
    out_dtype = out_dtype or x.dtype
    y = out if out is not None else torch.empty((rows, dim), dtype=out_dtype, device=dev)
    mul, add, mod_dt, mod_stride, split = _mod_args(mul, add, mul2, add2, dim, split)
    rpb = rows_per_batch or rows
    check(lib().difflet_rocm_layernorm_modulate(
        _ptr(x2), x2.stride(0), _ptr(y), y.stride(0), _dt(x2), _dt(y), rows, dim, _ptr(mul),
        _ptr(add), mod_dt, mod_stride, rpb, split, int(one_plus), float(eps), _stream(dev)),
        "layernorm_modulate")
    return y.reshape(*x.shape[:-1], dim) if out is None else y


def _mod_args(mul, add, mul2, add2, dim, split):
    """Kernel arguments for the modulation vectors: one set ([batches, dim]), or with split > 0
    two [dim] vectors per operand whose distance in elements becomes the batch stride."""
    if not split:
        return (*_mod_vectors(mul, add, dim), 0)
    for a, b2 in ((mul, mul2), (add, add2)):
        if (a is None) != (b2 is None):
            raise ValueError("split modulation: give both segments' vectors or neither")
    pairs = [(a, b2) for a, b2 in ((mul, mul2), (add, add2)) if a is not None]
    if not pairs:
        return None, None, _lib.F32, 0, int(split)
    dtype = pairs[0][0].dtype
    stride = None
    for a, b2 in pairs:
        if a.dtype != dtype or b2.dtype != dtype or a.numel() != dim or b2.numel() != dim or \
                a.stride(-1) != 1 or b2.stride(-1) != 1:
            raise ValueError("split modulation: [dim] vectors of one dtype with contiguous rows")
        d, r = divmod(b2.data_ptr() - a.data_ptr(), a.element_size())
        if r or (stride is not None and d != stride):
            raise ValueError("split modulation: both operands' second vectors must sit at one "
                             "distance from their first")
        stride = d
    return mul, add, _dt(pairs[0][0]), stride, int(split)


def _mod_vectors(mul, add, dim):
    """Modulation vectors as [batches, dim] rows sharing one batch stride, and their dtype."""
    mod = mul if mul is not None else add
    if mod is None:
        return None, None, _lib.F32, 0
    if mul is not None and add is not None and mul.dtype != add.dtype:
        add = add.to(mul.dtype)
    mul2 = mul.reshape(-1, dim) if mul is not None else None
    add2 = add.reshape(-1, dim) if add is not None else None
    for t in (mul2, add2):
        if t is not None and t.stride(-1) != 1:
            raise ValueError("modulation vectors must have contiguous rows")
    if mul2 is not None and add2 is not None and mul2.stride(0) != add2.stride(0):
        add2 = add2.contiguous()
        mul2 = mul2.contiguous()
    ref = mul2 if mul2 is not None else add2
    return mul2, add2, _dt(ref), (ref.stride(0) if ref.shape[0] > 1 else 0)


def layernorm_modulate_fp8(x: torch.Tensor, mul: torch.Tensor | None,
                           add: torch.Tensor | None, *, eps: float, one_plus: bool = True,
                           rows_per_batch: int | None = None, split: int = 0,
                           mul2: torch.Tensor | None = None, add2: torch.Tensor | None = None,
                           out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """layernorm_modulate rounded to bf16 and quantized per row to e4m3 in one pass:
    (codes float8_e4m3fn [rows, dim], scales fp32 [rows]), equal to quantize_fp8_rowwise of the
    bf16 layernorm_modulate output."""
    dev = _on_gpu(x)
    x2 = _rows2d(x, "layernorm_modulate_fp8")
    rows, dim = x2.shape
    if out is None:
        q = torch.empty((rows, dim), dtype=torch.float8_e4m3fn, device=dev)
        sc = torch.empty((rows,), dtype=torch.float32, device=dev)
    else:
        q, sc = out
        if q.element_size() != 1 or sc.dtype != torch.float32 or q.shape[0] != rows or \
                q.shape[-1] < dim or sc.numel() < rows or not sc.is_contiguous():
            raise ValueError("layernorm_modulate_fp8: out must be (8-bit [rows, >=dim], "
                             "contiguous fp32 [rows])")
    mul, add, mod_dt, mod_stride, split = _mod_args(mul, add, mul2, add2, dim, split)
    rpb = rows_per_batch or rows
    check(lib().difflet_rocm_layernorm_modulate_fp8(
        _ptr(x2), x2.stride(0), _ptr(q), q.stride(0), _ptr(sc), _dt(x2), rows, dim, _ptr(mul),
        _ptr(add), mod_dt, mod_stride, rpb, split, int(one_plus), float(eps), _stream(dev)),
        "layernorm_modulate_fp8")
    return q, sc


def layernorm_modulate_mx(x: torch.Tensor, mul: torch.Tensor | None,
                          add: torch.Tensor | None, *, eps: float, one_plus: bool = True,
                          rows_per_batch: int | None = None, split: int = 0,
                          mul2: torch.Tensor | None = None, add2: torch.Tensor | None = None,
                          out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """layernorm_modulate rounded to bf16 and quantized to MXFP8 in the GEMM's swizzled layout in
    one pass: (codes float8_e4m3fn [rows, dim], E8M0 scales uint8 [rows, dim / 32]), equal to
    quantize_mxfp8(swizzled=True) of the bf16 layernorm_modulate output. x bf16, dim a multiple
    of 512."""
    dev = _on_gpu(x)
    x2 = _rows2d(x, "layernorm_modulate_mx")
    rows, dim = x2.shape
    if x2.dtype != torch.bfloat16 or dim % 512:
        raise ValueError(f"layernorm_modulate_mx: x must be bf16 with a width that is a "
                         f"multiple of 512, got {x2.dtype} [{rows}, {dim}]")
    if out is None:
        q = torch.empty((rows, dim), dtype=torch.float8_e4m3fn, device=dev)
        sc = torch.empty((rows, dim // 32), dtype=torch.uint8, device=dev)
    else:
        q, sc = out
        if q.element_size() != 1 or sc.dtype != torch.uint8 or q.shape[0] != rows or \
                sc.shape[0] != rows or q.shape[-1] < dim or sc.shape[-1] < dim // 32 or \
                q.stride(-1) != 1 or sc.stride(-1) != 1:
            raise ValueError("layernorm_modulate_mx: out must be (8-bit [rows, >=dim], "
                             "uint8 [rows, >=dim / 32]), unit column stride")
    mul, add, mod_dt, mod_stride, split = _mod_args(mul, add, mul2, add2, dim, split)
    rpb = rows_per_batch or rows
    check(lib().difflet_rocm_layernorm_modulate_mx(
        _ptr(x2), x2.stride(0), _ptr(q), q.stride(0), _ptr(sc), sc.stride(0), _dt(x2), rows, dim,
        _ptr(mul), _ptr(add), mod_dt, mod_stride, rpb, split, int(one_plus), float(eps),
        _stream(dev)), "layernorm_modulate_mx")
    return q, sc


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    dev = _on_gpu(x)
    x2 = _rows2d(x, "rms_norm")
    rows, dim = x2.shape
    y = torch.empty((rows, dim), dtype=x.dtype, device=dev)
    if rows == 0:
        return y.reshape(x.shape)
    wdt = _dt(weight) if weight is not None else _lib.F32
    check(lib().difflet_rocm_rms_norm(_ptr(x2), x2.stride(0), _ptr(y), dim, _dt(x2), rows, dim,
                                      _ptr(weight), wdt, float(eps), _stream(dev)), "rms_norm")
    return y.reshape(x.shape)


def qk_norm_rope(buf: torch.Tensor, *, heads: int, head_dim: int, q_off: int, k_off: int,
                 wq: torch.Tensor | None, wk: torch.Tensor | None, eps: float,
                 cos: torch.Tensor | None, sin: torch.Tensor | None, law: int = 0,
                 do_norm: bool | int = True, split: int = 0, wq2: torch.Tensor | None = None,
                 wk2: torch.Tensor | None = None) -> None:
    """In place on a [rows, ld] projection buffer: RMSNorm of q (columns q_off + h * head_dim ..;
    q_off < 0 skips q) and k, per head (do_norm True / 1) or over all heads of the row (2), then
    the rotary embedding with fp32 tables [S, head_dim] (cos None skips it). With split > 0,
    rows >= split use the weights wq2 / wk2."""
    if split and ((wq2 is None) != (wq is None) or (wk2 is None) != (wk is None)):
        raise ValueError("qk_norm_rope: split needs second weights wherever there are first")
    dev = _on_gpu(buf)
    if buf.dim() != 2 or buf.stride(1) != 1:
        raise ValueError("qk_norm_rope: buf must be 2-D with contiguous rows")
    rows = buf.shape[0]
    wdt = _dt(wq) if wq is not None else (_dt(wk) if wk is not None else _lib.F32)
    if cos is not None:
        if cos.dtype != torch.float32 or sin.dtype != torch.float32:
            raise TypeError("rope tables must be fp32")
        cos, sin = cos.contiguous(), sin.contiguous()
    for w2 in (wq2, wk2):
        if split and w2 is not None and _dt(w2) != wdt:
            raise TypeError("qk_norm_rope: both segments' weights share one dtype")
    check(lib().difflet_rocm_qk_norm_rope(
        _ptr(buf), buf.stride(0), _dt(buf), rows, heads, head_dim, q_off, k_off, int(do_norm),
        _ptr(wq), _ptr(wk), int(split), _ptr(wq2), _ptr(wk2), wdt, float(eps), _ptr(cos),
        _ptr(sin), cos.shape[0] if cos is not None else 0, law, _stream(dev)), "qk_norm_rope")


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, *, law: int) -> torch.Tensor:
    """Rotary embedding of x [..., S, D] with fp32 tables [S, D] (law 0: fp32 interleaved,
    law 1: stride-2 with cos of the even and sin of the odd entries)."""
    dev = _on_gpu(x, cos, sin)
    s, d = x.shape[-2], x.shape[-1]
    xv = x.reshape(-1, s, d)
    if xv.stride(-1) != 1:
        xv = xv.contiguous()
    y = torch.empty(xv.shape, dtype=x.dtype, device=dev)
    c = cos.reshape(-1, d).to(torch.float32).contiguous()
    sn = sin.reshape(-1, d).to(torch.float32).contiguous()
    check(lib().difflet_rocm_rope(_ptr(xv), _ptr(y), _dt(xv), xv.shape[0], s, d, xv.stride(0),
                                  xv.stride(1), y.stride(0), y.stride(1), _ptr(c), _ptr(sn),
                                  c.shape[0], law, _stream(dev)), "rope")
    return y.reshape(x.shape)


# ------------------------------------------------------------------------ small kernels
def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    dev = _on_gpu(x)
    xc = x.contiguous()
    y = torch.empty_like(xc)
    check(lib().difflet_rocm_gelu_tanh(_ptr(xc), _ptr(y), _dt(xc), xc.numel(), _stream(dev)),
          "gelu_tanh")
    return y


def gate_residual(residual: torch.Tensor, x: torch.Tensor, gate: torch.Tensor, *,
                  rows_per_batch: int | None = None) -> torch.Tensor:
    """residual + gate * x with gate [dim] or [batches, dim]."""
    dev = _on_gpu(residual, x, gate)
    r2 = residual.reshape(-1, residual.shape[-1]).contiguous()
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    g2 = gate.reshape(-1, gate.shape[-1]).contiguous()
    y = torch.empty_like(r2)
    check(lib().difflet_rocm_gate_residual(_ptr(r2), _ptr(x2), _ptr(g2), _ptr(y), _dt(r2),
                                           _dt(g2), r2.shape[0], r2.shape[1],
                                           g2.stride(0) if g2.shape[0] > 1 else 0,
                                           rows_per_batch or r2.shape[0], _stream(dev)),
          "gate_residual")
    return y.reshape(residual.shape)


def gemv(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None, *,
         act: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """act(x) W^T + b for x [m <= 8, K] (act 1 = SiLU on x), W bf16 [N, K]."""
    dev = _on_gpu(x, w)
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    m, k = x2.shape
    n = w.shape[0]
    if w.dtype != torch.bfloat16 or w.stride(1) != 1:
        raise TypeError("gemv weights must be bf16 with contiguous rows")
    if bias is not None and bias.dtype != x2.dtype:
        bias = bias.to(x2.dtype)
    y = out if out is not None else torch.empty((m, n), dtype=x2.dtype, device=dev)
    check(lib().difflet_rocm_gemv(_ptr(x2), _dt(x2), m, k, x2.stride(0), _ptr(w), w.stride(0), n,
                                  _ptr(bias), _ptr(y), y.stride(0), int(act), _stream(dev)),
          "gemv")
    return y


def timestep_embedding(t: torch.Tensor, dim: int, *, flip_sin_to_cos: bool,
                       downscale_freq_shift: float, scale: float = 1.0,
                       max_period: float = 10000.0, dtype: torch.dtype = torch.float32
                       ) -> torch.Tensor:
    dev = _on_gpu(t)
    tt = t.reshape(-1).to(torch.float32).contiguous()
    y = torch.empty((tt.shape[0], dim), dtype=dtype, device=dev)
    check(lib().difflet_rocm_timestep_embedding(_ptr(tt), _ptr(y), _dt(y), tt.shape[0], dim,
                                                int(flip_sin_to_cos),
                                                float(downscale_freq_shift), float(scale),
                                                float(max_period), _stream(dev)),
          "timestep_embedding")
    return y


# ------------------------------------------------------------------------ text encoders
def gemm_bf16_f32out(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """A W^T for bf16 a [M, K] and w [N, K] (K a multiple of 64) on the bf16 matrix cores, the
    fp32 accumulators stored as they are: [M, N] fp32 (a view of [M, N rounded up to 4], w's
    missing rows zero). The VAE decoders' mid-block attention scores."""
    m, k = a.shape
    n = w.shape[0]
    npad = -(-n // 4) * 4
    if npad != n:
        w2 = torch.zeros(npad, k, dtype=w.dtype, device=w.device)
        w2[:n] = w
        w = w2
    y = torch.empty(m, npad, dtype=torch.float32, device=a.device)
    gemm_grouped([Problem(a, w, y)], kind="bf16", epilogue=_lib.EPI_F32)
    return y[:, :n]


def gemm_f32(a: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None, *,
             residual: torch.Tensor | None = None, out: torch.Tensor | None = None
             ) -> torch.Tensor:
    """A W^T (+ bias) (+ residual) in fp32 on the matrix cores: a [M, K], w [N, K], bias [N],
    residual and out [M, N] (residual may be out). K and N multiples of 4."""
    for name, t in (("a", a), ("w", w), ("bias", bias), ("residual", residual), ("out", out)):
        if t is not None and t.dtype != torch.float32:
            raise TypeError(f"gemm_f32: {name} must be fp32, got {t.dtype}")
    if a.dim() != 2 or w.dim() != 2 or a.shape[1] != w.shape[1]:
        raise ValueError(f"gemm_f32: a {tuple(a.shape)} and w {tuple(w.shape)} do not chain")
    m, k = a.shape
    n = w.shape[0]
    if k % 4 or n % 4:
        raise ValueError(f"gemm_f32: K ({k}) and N ({n}) must be multiples of 4")
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != n or bias.stride(0) != 1):
        raise ValueError(f"gemm_f32: bias must be a contiguous [{n}] vector")
    for name, t in (("residual", residual), ("out", out)):
        if t is not None and (t.dim() != 2 or tuple(t.shape) != (m, n) or t.stride(1) != 1):
            raise ValueError(f"gemm_f32: {name} must be [{m}, {n}] with contiguous rows")
    dev = _on_gpu(a, w, bias, residual, out)
    a2 = a if a.stride(1) == 1 and a.stride(0) % 4 == 0 else a.contiguous()
    w2 = w if w.stride(1) == 1 and w.stride(0) % 4 == 0 else w.contiguous()
    y = out if out is not None else torch.empty((m, n), dtype=torch.float32, device=dev)
    check(lib().difflet_rocm_gemm_f32(_ptr(a2), a2.stride(0), _ptr(w2), w2.stride(0), _ptr(bias),
                                      _ptr(residual),
                                      residual.stride(0) if residual is not None else 0,
                                      _ptr(y), y.stride(0), m, n, k, _stream(dev)), "gemm_f32")
    return y


def gated_gelu(x: torch.Tensor, f: int, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """gelu_tanh(x[:, :f]) * x[:, f:2f] for x [rows, >= 2f] with contiguous rows."""
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < 2 * f:
        raise ValueError(f"gated_gelu: x must be [rows, >= {2 * f}] with contiguous rows")
    dev = _on_gpu(x, out)
    y = out if out is not None else torch.empty((x.shape[0], f), dtype=x.dtype, device=dev)
    if y.dtype != x.dtype or tuple(y.shape) != (x.shape[0], f) or y.stride(1) != 1:
        raise ValueError("gated_gelu: out must match x's dtype and be [rows, f]")
    check(lib().difflet_rocm_gated_gelu(_ptr(x), x.stride(0), _ptr(y), y.stride(0), _dt(x),
                                        x.shape[0], f, _stream(dev)), "gated_gelu")
    return y


def embedding(ids: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """table[ids] for int64 ids (any shape) and a [rows, dim] table with contiguous rows. Ids
    outside [0, rows) raise IndexError, as F.embedding does (checked before the gather)."""
    if ids.dtype != torch.int64:
        raise TypeError(f"embedding: ids must be int64, got {ids.dtype}")
    if table.dim() != 2 or table.stride(1) != 1:
        raise ValueError("embedding: table must be [rows, dim] with contiguous rows")
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= table.shape[0]):
        raise IndexError(f"embedding: ids outside [0, {table.shape[0]})")
    dev = _on_gpu(table)
    flat = ids.reshape(-1).to(dev).contiguous()
    es = table.element_size()
    y = torch.empty((flat.shape[0], table.shape[1]), dtype=table.dtype, device=dev)
    check(lib().difflet_rocm_embedding(_ptr(flat), flat.shape[0], _ptr(table), table.shape[0],
                                       table.stride(0) * es, _ptr(y), y.stride(0) * es,
                                       table.shape[1] * es, _stream(dev)), "embedding")
    return y.reshape(*ids.shape, table.shape[1])


def relative_bias(buckets: torch.Tensor, table: torch.Tensor, *, batch: int, seq_q: int,
                  seq_k: int, key_keep: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [batch, heads, seq_q, seq_k] T5 position bias: table[buckets[k - q + seq_q - 1]]
    per head (table [num_buckets, heads]); keys with key_keep[b, k] == 0 get the lowest float.
    buckets: int32 [seq_q + seq_k - 1], values in [0, num_buckets)."""
    if buckets.dtype != torch.int32 or buckets.dim() != 1 or buckets.shape[0] != seq_q + seq_k - 1:
        raise ValueError(f"relative_bias: buckets must be int32 [{seq_q + seq_k - 1}]")
    if table.dim() != 2 or not table.is_contiguous():
        raise ValueError("relative_bias: table must be a contiguous [num_buckets, heads]")
    if key_keep is not None and (tuple(key_keep.shape) != (batch, seq_k)
                                 or key_keep.dtype not in (torch.bool, torch.uint8)):
        raise ValueError(f"relative_bias: key_keep must be bool/uint8 [{batch}, {seq_k}]")
    dev = _on_gpu(buckets, table, key_keep)
    keep = None
    if key_keep is not None:
        keep = key_keep.contiguous()
        keep = keep.view(torch.uint8) if keep.dtype == torch.bool else keep
    nb, heads = table.shape
    y = torch.empty((batch, heads, seq_q, seq_k), dtype=torch.float32, device=dev)
    check(lib().difflet_rocm_relative_bias(_ptr(buckets.contiguous()), nb, _ptr(table), _dt(table),
                                           heads, batch, seq_q, seq_k, _ptr(keep),
                                           keep.stride(0) if keep is not None else 0, _ptr(y),
                                           _stream(dev)), "relative_bias")
    return y


# ------------------------------------------------------------------------ VAE decoder
_GN_WORKSPACE: dict[tuple[int, int], torch.Tensor] = {}


def group_norm(x: torch.Tensor, groups: int, weight: torch.Tensor | None,
               bias: torch.Tensor | None, eps: float, *, silu: bool = False,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """GroupNorm (+ SiLU) of channels-last x [batch, pixels, C] (bf16 or fp32) with fp32 affine
    vectors; statistics in fp32 / double, two passes."""
    if x.dim() != 3 or not x.is_contiguous():
        raise ValueError("group_norm: x must be a contiguous [batch, pixels, channels]")
    b, p, c = x.shape
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None and (t.dtype != torch.float32 or t.shape != (c,) or not t.is_contiguous()):
            raise ValueError(f"group_norm: {name} must be a contiguous fp32 [{c}]")
    if c % groups or c % 8:
        raise ValueError(f"group_norm: {c} channels are not a multiple of 8 and of {groups} groups")
    dev = _on_gpu(x, weight, bias, out)
    y = out if out is not None else torch.empty_like(x)
    need = int(lib().difflet_rocm_group_norm_workspace_bytes(b, p, c, groups))
    # one workspace per (device, stream), as for the GEMM and attention workspaces: launches on
    # one stream run in order and can share it, and a grown one replaces the old on the stream
    # that allocated it, so the allocator reuses the old block only after its last reader
    i = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (i, torch.cuda.current_stream(torch.device("cuda", i)).cuda_stream)
    ws = _GN_WORKSPACE.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=torch.device("cuda", i))
        _GN_WORKSPACE[key] = ws
    check(lib().difflet_rocm_group_norm(_ptr(x), _ptr(y), _dt(x), b, p, c, groups, _ptr(weight),
                                        _ptr(bias), float(eps), int(bool(silu)), _ptr(ws),
                                        ws.numel(), _stream(dev)), "group_norm")
    return y


def im2col3x3(x: torch.Tensor, *, upsample: bool = False, kpad: int | None = None,
              row0: int = 0, rows: int | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """[H, W, C] channels-last image -> [rows, kpad] rows of the 9 taps' channels around output
    pixels row0 .. row0 + rows - 1 (all by default; zero padding, and nearest 2x upsampling
    first when upsample)."""
    if x.dim() != 3 or not x.is_contiguous():
        raise ValueError("im2col3x3: x must be a contiguous [height, width, channels]")
    h, w, c = x.shape
    ev = 4 if x.dtype == torch.float32 else 8
    kpad = kpad if kpad is not None else -(-9 * c // ev) * ev
    dev = _on_gpu(x, out)
    up = int(bool(upsample))
    total = (h << up) * (w << up)
    rows = total - row0 if rows is None else rows
    y = out if out is not None else torch.empty((rows, kpad), dtype=x.dtype, device=dev)
    if y.dtype != x.dtype or y.shape[0] != rows or y.shape[1] < kpad or y.stride(1) != 1:
        raise ValueError(f"im2col3x3: out must be [{rows}, >= {kpad}] of x's dtype")
    check(lib().difflet_rocm_im2col3x3(_ptr(x), _dt(x), h, w, c, up, row0, rows, _ptr(y),
                                       y.stride(0), kpad, _stream(dev)), "im2col3x3")
    return y


def softmax_rows(s: torch.Tensor, scale: float, *, dtype: torch.dtype = torch.float32,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(s * scale) over the last dim of fp32 scores [rows, cols], written in dtype."""
    if s.dtype != torch.float32 or s.dim() != 2 or s.stride(1) != 1:
        raise ValueError("softmax_rows: s must be fp32 [rows, cols] with contiguous rows")
    dev = _on_gpu(s, out)
    p = out if out is not None else torch.empty(s.shape, dtype=dtype, device=dev)
    check(lib().difflet_rocm_softmax_rows(_ptr(s), s.stride(0), _ptr(p), p.stride(0), _dt(p),
                                          s.shape[0], s.shape[1], float(scale), _stream(dev)),
          "softmax_rows")
    return p


# ------------------------------------------------------------------------ Wan's 3D VAE decoder
def conv_causal(x: torch.Tensor, hw: tuple[int, int], channels: int, frames: int, w: torch.Tensor,
                bias: torch.Tensor | None = None, *, kt: int, ks: int, upsample: bool = False,
                lead_frames: int = 0, frames_per_block: int = 1, frame_stride: int | None = None,
                sub_stride: int = 0, pixel_stride: int | None = None,
                residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
                split: bool = True) -> torch.Tensor:
    """The causal (kt, ks, ks) convolution of `frames` chunk frames as one implicit GEMM (bf16
    on the bf16 matrix cores, fp32 on the fp32 GEMM):
    [frames * Ho * Wo, n] = the im2col rows of im2col_causal times w [n, kpad] (+ bias, +
    residual), without writing the rows. x holds the frames (contiguous; buffer frame b at
    element (b // frames_per_block) * frame_stride + (b % frames_per_block) * sub_stride, pixels
    pixel_stride apart); chunk frame f is buffer frame f + lead_frames, so a causal convolution
    passes [cache frame -2, cache frame -1, frames...] with lead_frames 2. split: a convolution
    too small to fill the device may cut its K stages (fp32 partial sums through a per-stream
    workspace); False runs whole tiles, bit-identical to the im2col rows' GEMM."""
    h, wd = hw
    if not x.is_contiguous():
        raise ValueError("conv_causal: x must be contiguous")
    if x.dtype not in (torch.bfloat16, torch.float32) or w.dtype != x.dtype:
        raise ValueError("conv_causal: bf16 or fp32 frames, and a weight of their dtype")
    pix = h * wd
    ld = channels if pixel_stride is None else pixel_stride
    fs = pix * ld if frame_stride is None else frame_stride
    up = int(bool(upsample))
    rows = frames * (h << up) * (wd << up)
    n, kpad = w.shape
    if w.stride(1) != 1 or w.stride(0) != kpad:
        raise ValueError("conv_causal: w must be a contiguous [n, kpad]")
    if frames > 0:
        last = frames - 1 + lead_frames
        end = ((last // frames_per_block) * fs + (last % frames_per_block) * sub_stride
               + (pix - 1) * ld + channels)
        if end > x.numel() or channels > ld:
            raise ValueError(f"conv_causal: buffer frames 0..{last} of {h}x{wd}x{channels} "
                             f"overrun x ({x.numel()} elements)")
    dev = _on_gpu(x, w, bias, residual, out)
    y = out if out is not None else torch.empty((rows, n), dtype=x.dtype, device=dev)
    if y.dtype != x.dtype or y.shape[0] != rows or y.shape[1] < n or y.stride(1) != 1:
        raise ValueError(f"conv_causal: out must be [{rows}, >= {n}] of x's dtype")
    if residual is not None and (residual.dtype != x.dtype or residual.shape[0] != rows
                                 or residual.shape[1] < n or residual.stride(1) != 1):
        raise ValueError(f"conv_causal: residual must be [{rows}, >= {n}] of x's dtype")
    if bias is not None and (bias.dtype != x.dtype or bias.numel() < n or not bias.is_contiguous()):
        raise ValueError(f"conv_causal: bias must hold {n} values of x's dtype")
    ws = None
    if split and rows and x.dtype == torch.bfloat16:
        i = dev.index if dev.index is not None else torch.cuda.current_device()
        with torch.cuda.device(i):
            need = int(lib().difflet_rocm_conv_causal_workspace_bytes(rows, n, kpad))
        if need:  # per (device, stream), as the group-norm workspace
            key = (i, torch.cuda.current_stream(torch.device("cuda", i)).cuda_stream)
            ws = _CONV_WORKSPACE.get(key)
            if ws is None or ws.numel() < need:
                ws = torch.empty(need, dtype=torch.uint8, device=torch.device("cuda", i))
                _CONV_WORKSPACE[key] = ws
    check(lib().difflet_rocm_conv_causal(
        _ptr(x), x.numel(), fs, frames_per_block, sub_stride, ld, lead_frames, _dt(x), h, wd,
        channels, kt, ks, up, frames, _ptr(w), n, kpad, _ptr(bias), _ptr(residual),
        0 if residual is None else residual.stride(0), _ptr(y), y.stride(0), _ptr(ws),
        0 if ws is None else ws.numel(), _stream(dev)), "conv_causal")
    return y


_CONV_WORKSPACE: dict[tuple[int, int], torch.Tensor] = {}


def im2col_causal(x: torch.Tensor, hw: tuple[int, int], channels: int, *, kt: int, ks: int,
                  kpad: int, upsample: bool = False, cache: torch.Tensor | None = None,
                  frames_per_block: int = 1, frame_stride: int | None = None,
                  sub_stride: int = 0, pixel_stride: int | None = None, row0: int = 0,
                  rows: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Rows of a causal (kt, ks, ks) convolution over the frames held in x (contiguous; frame f
    at element (f // frames_per_block) * frame_stride + (f % frames_per_block) * sub_stride,
    pixels pixel_stride apart; by default [frames, H * W, channels]), frames -2 and -1 from
    cache [2, H * W, channels] (zeros when None): [rows, kpad], output rows row0 .. row0 + rows
    - 1 (default: every frame of x) at the (upsampled) output resolution."""
    h, w = hw
    if not x.is_contiguous():
        raise ValueError("im2col_causal: x must be contiguous")
    pix = h * w
    ld = channels if pixel_stride is None else pixel_stride
    fpb = frames_per_block
    fs = pix * ld if frame_stride is None else frame_stride
    up = int(bool(upsample))
    po = (h << up) * (w << up)
    if rows is None:
        if frame_stride is not None or fpb != 1:
            raise ValueError("im2col_causal: give rows when the frames are strided")
        rows = (x.numel() // (pix * ld)) * po - row0
    dev = _on_gpu(x, cache, out)
    if row0 < 0 or rows < 0:
        raise ValueError("im2col_causal: bad row range")
    if rows:
        # every element the rows read lies inside x (and cache)
        last = (row0 + rows - 1) // po
        end = (last // fpb) * fs + (last % fpb) * sub_stride + (pix - 1) * ld + channels
        if end > x.numel() or channels > ld:
            raise ValueError(f"im2col_causal: frames 0..{last} of {h}x{w}x{channels} overrun x "
                             f"({x.numel()} elements)")
    if cache is not None and (cache.dtype != x.dtype or tuple(cache.shape) != (2, pix, channels)
                              or not cache.is_contiguous()):
        raise ValueError(f"im2col_causal: cache must be a contiguous [2, {pix}, {channels}] of "
                         "x's dtype")
    y = out if out is not None else torch.empty((rows, kpad), dtype=x.dtype, device=dev)
    if y.dtype != x.dtype or y.shape[0] != rows or y.shape[1] < kpad or y.stride(1) != 1:
        raise ValueError(f"im2col_causal: out must be [{rows}, >= {kpad}] of x's dtype")
    check(lib().difflet_rocm_im2col_causal(_ptr(x), fs, fpb, sub_stride, ld, _ptr(cache), _dt(x),
                                           h, w, channels, kt, ks, up, row0, rows, _ptr(y),
                                           y.stride(0), kpad, _stream(dev)), "im2col_causal")
    return y


def rms_norm_channels(x: torch.Tensor, gamma: torch.Tensor, *, eps: float = 1e-12,
                      silu: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """WanRMSNorm over the last dim of rows x [rows, C] (bf16 or fp32, unit stride along C):
    x sqrt(C) / max(||x||, eps) * gamma (fp32 [C]), then SiLU when silu."""
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("rms_norm_channels: x must be [rows, channels] with unit column stride")
    rows, c = x.shape
    if gamma.dtype != torch.float32 or gamma.numel() != c or not gamma.is_contiguous():
        raise ValueError(f"rms_norm_channels: gamma must be a contiguous fp32 [{c}]")
    dev = _on_gpu(x, gamma, out)
    y = out if out is not None else torch.empty_like(x)
    if y.shape != x.shape or y.dtype != x.dtype or y.stride(1) != 1:
        raise ValueError("rms_norm_channels: out must match x")
    check(lib().difflet_rocm_rms_norm_channels(_ptr(x), x.stride(0), _ptr(y), y.stride(0), _dt(x),
                                               rows, c, _ptr(gamma), float(eps), int(bool(silu)),
                                               _stream(dev)), "rms_norm_channels")
    return y


def rows_to_planes(x: torch.Tensor, channels: int, *, lo: float = float("-inf"),
                   hi: float = float("inf"), out: torch.Tensor | None = None) -> torch.Tensor:
    """[n, >= channels] rows -> [channels, n] planes, clamped to [lo, hi]."""
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] < channels:
        raise ValueError(f"rows_to_planes: x must be [n, >= {channels}] with unit column stride")
    n = x.shape[0]
    dev = _on_gpu(x, out)
    y = out if out is not None else torch.empty((channels, n), dtype=x.dtype, device=dev)
    if y.dtype != x.dtype or y.numel() != channels * n or not y.is_contiguous():
        raise ValueError(f"rows_to_planes: out must be a contiguous [{channels}, {n}] of x's dtype")
    check(lib().difflet_rocm_rows_to_planes(_ptr(x), x.stride(0), _dt(x), n, channels, _ptr(y),
                                            float(lo), float(hi), _stream(dev)), "rows_to_planes")
    return y
