"""Device linear layers of the fused DiT blocks: one weight in the layout its GEMM reads.

kind "bf16": W bf16 [N, K].
kind "fp8" : per-output-channel e4m3 codes [N, K] + fp32 scales [N]; activations are quantized
             per token right before the GEMM (difflet_rocm_quantize_fp8_rowwise), and the GEMM
             applies s_x[m] * s_w[n] in its epilogue.
kind "mx"  : MXFP8, codes in swizzle order [N, K] + E8M0 scales [N, K/32] (the block law of
             difflet/quant/mx.py:46-108); activations quantized per call in the same order.
"""

from __future__ import annotations

import torch

from difflet_amd import kernels
from difflet_amd.kernels import Problem

KINDS = ("bf16", "fp8", "mx")


class DeviceLinear:
    __slots__ = ("kind", "w", "ws", "bias", "n", "k")

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, kind: str = "bf16"):
        if kind not in KINDS:
            raise ValueError(f"linear kind must be one of {KINDS}, got {kind!r}")
        w = weight.to(torch.bfloat16).contiguous()
        self.kind = kind
        self.n, self.k = w.shape
        self.bias = None if bias is None else bias.to(device=w.device, dtype=torch.bfloat16).contiguous()
        if kind == "bf16":
            self.w, self.ws = w, None
        elif kind == "fp8":
            self.w, self.ws = kernels.quantize_fp8_rowwise(w)
        else:
            self.w, self.ws = kernels.quantize_mxfp8(w, swizzled=True)

    @classmethod
    def from_fp8(cls, codes: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None,
                 kind: str) -> "DeviceLinear":
        """A linear from stored codes and scales (a quantized checkpoint), with no quantization:
        kind "fp8": codes [N, K] + fp32 scales [N]; kind "mx": codes [N, K] in logical K order +
        uint8 E8M0 scales [N, K/32], the codes gathered into the swizzle order the GEMM reads
        (a permutation of bytes within each row)."""
        from difflet_amd.quant.linear import _swizzle_index

        if kind not in ("fp8", "mx"):
            raise ValueError(f"stored codes are kind 'fp8' or 'mx', got {kind!r}")
        if codes.dtype != torch.float8_e4m3fn or codes.dim() != 2:
            raise ValueError(f"codes must be float8_e4m3fn [N, K], got {codes.dtype} {list(codes.shape)}")
        n, k = codes.shape
        want = ((n,), torch.float32) if kind == "fp8" else ((n, k // 32), torch.uint8)
        if tuple(scale.shape) != want[0] or scale.dtype != want[1]:
            raise ValueError(f"kind {kind!r} scales are {want[1]} {list(want[0])}, got "
                             f"{scale.dtype} {list(scale.shape)}")
        self = cls.__new__(cls)
        self.kind, self.n, self.k = kind, n, k
        if kind == "mx":
            idx = _swizzle_index(k, codes.device)
            codes = codes.view(torch.uint8)[:, idx].view(torch.float8_e4m3fn)
        self.w, self.ws = codes.contiguous(), scale.contiguous()
        self.bias = None if bias is None else bias.to(device=codes.device, dtype=torch.bfloat16).contiguous()
        return self

    def rows_in_swizzle_order(self) -> "DeviceLinear":
        """This linear with its output rows (weight rows, scales, bias) gathered into the MXFP8
        swizzle order over N (difflet/quant/mx.py:65-76): its GEMM then writes output column p
        as logical column perm[p], the layout in which the GELU -> MXFP8 epilogue's codes are
        the next MXFP8 GEMM's A operand."""
        from difflet_amd.quant.linear import _swizzle_index

        if self.kind != "mx" or self.n % 32:
            raise ValueError("rows in swizzle order: an MXFP8 linear with N % 32 == 0")
        idx = _swizzle_index(self.n, self.w.device)
        out = DeviceLinear.__new__(DeviceLinear)
        out.kind, out.n, out.k = self.kind, self.n, self.k
        out.w = self.w.view(torch.uint8)[idx].view(self.w.dtype).contiguous()
        out.ws = self.ws[idx].contiguous()
        out.bias = None if self.bias is None else self.bias[idx].contiguous()
        return out

    def prep(self, a: torch.Tensor, gelu_from: int | None = None
             ) -> tuple[torch.Tensor, torch.Tensor | None]:
        """The GEMM's A operand for activations a [M, K] (quantized for the fp8 kinds).
        gelu_from (fp8 only): a's columns from there on are an MLP pre-activation, quantized as
        bf16(gelu_tanh(a)) (the per-token fp8 law's GELU point)."""
        if self.kind == "bf16":
            return a, None
        if self.kind == "fp8":
            return kernels.quantize_fp8_rowwise(a, gelu_from=gelu_from)
        if gelu_from is not None:
            raise ValueError("the GELU-at-quantization point is part of the per-token fp8 law")
        return kernels.quantize_mxfp8(a, swizzled=True)

    def problem(self, a: torch.Tensor, c: torch.Tensor, *, gate=None, residual=None,
                prepared=None, norm_q=None, norm_k=None, rope_row0: int = 0,
                c_scale=None) -> Problem:
        aq, asc = prepared if prepared is not None else self.prep(a)
        return Problem(aq, self.w, c, self.bias, gate, residual, asc, self.ws,
                       norm_q=norm_q, norm_k=norm_k, rope_row0=rope_row0, c_scale=c_scale)

    def __call__(self, a: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        c = out if out is not None else torch.empty((a.shape[0], self.n), dtype=torch.bfloat16,
                                                    device=a.device)
        run([self.problem(a, c)], self.kind)
        return c

    def weight_bytes(self) -> int:
        b = self.w.numel() * self.w.element_size()
        if self.ws is not None:
            b += self.ws.numel() * self.ws.element_size()
        return b


def linear_group(get, q, prefixes: list[str], kind: str, *,
           along_k: bool = False, bias_prefix: str | None = None) -> DeviceLinear:
    """One device linear over the linears at ``prefixes``, their weights concatenated along N
    (rows) or, ``along_k``, along K (the single block's proj_out halves, bias ``bias_prefix``).

    Without a quantized checkpoint ``q`` the dense weights are quantized here by ``kind``. With
    one, the group's stored fp8 codes and scales are loaded as they are (every member of a group
    stored quantized, or none: then the dense weights run in bf16)."""
    cat_dim = 1 if along_k else 0
    bias_names = [bias_prefix] if along_k else prefixes
    bias = torch.cat([get(f"{p}.bias") for p in bias_names], dim=0)
    if q is not None:
        parts = [q.fp8(p) for p in prefixes]
        stored = [p is not None for p in parts]
        if all(stored):
            lk = "fp8" if q.format == "fp8_rowwise" else "mx"
            if along_k and (lk == "fp8" or parts[0][0].shape[1] % 512):
                raise ValueError(f"{prefixes}: stored halves fuse along K only as MXFP8 with the "
                                 "first half's K a multiple of 512 (the swizzle tile)")
            dev = bias.device
            codes = torch.cat([c.to(dev) for c, _ in parts], dim=cat_dim)
            scales = torch.cat([sc.to(dev) for _, sc in parts], dim=cat_dim)
            return DeviceLinear.from_fp8(codes, scales, bias, lk)
        if any(stored):
            raise ValueError(f"{prefixes}: one GEMM runs these linears, so they are stored "
                             "quantized all together or not at all")
        kind = "bf16"
    w = torch.cat([get(f"{p}.weight") for p in prefixes], dim=cat_dim)
    return DeviceLinear(w, bias, kind)


def run(problems, kind: str, epilogue: int = 0, act_col_start: int = 0, qk=None) -> None:
    # the stream's split workspace: the kernels cut a launch's last wave of tiles along K where
    # that pays (Qwen-Image's 336-tile projections) and run every other launch as whole tiles
    kernels.gemm_grouped(problems, kind=kind, epilogue=epilogue, act_col_start=act_col_start,
                         qk=qk, workspace="shared")
