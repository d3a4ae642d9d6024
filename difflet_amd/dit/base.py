"""Launch helpers shared by the fused DiT steps, and the joint (dual-stream) block they share.

The FLUX double-stream block (difflet/models/flux/modeling_flux.py:796-867) and the Qwen-Image
block (difflet/models/qwen_image/modeling_qwen.py:107-285) run the same sequence: per stream
LayerNorm + modulation (shift, scale, gate twice), q/k/v projections, per-head q/k RMSNorm and
RoPE, one joint attention over [text | image], output projections with gate * (x + bias) +
residual, then per stream LayerNorm + modulation and a GELU-tanh MLP with the same gated
residual. On the device each step is one launch for both streams (grouped GEMMs over the text
and image row ranges of one [S, ...] buffer).

Buffers (batch 1, S = S_txt + S_img, D = hidden, text rows first):
  h [S, D] residual stream, n [S, D] modulated LayerNorm output, qkv [S, 3D], ff [S, mlp];
  fp8 steps add nq [S, D] e4m3 codes and ns [S] scales written by the fused LayerNorm; MXFP8
  steps add nq [S, D] codes in the GEMM's swizzled order and nsx [S, D / 32] E8M0 scales.
"""

from __future__ import annotations

import contextlib
import math

import torch

from difflet_amd import _lib, kernels
from difflet_amd.dit.linear import run

EPS = 1e-6
_NULL = contextlib.nullcontext()


class JointDiT:
    """Mixin: needs self.cfg (hidden, heads, head_dim, mlp), self.kind, self.device and
    self.probe (None, or probe(name) -> context manager timing one launch)."""

    def _mods(self, mod: torch.Tensor, off: int, n: int):
        d = self.cfg.hidden
        return [mod[:, off + j * d: off + (j + 1) * d] for j in range(n)]

    def _timed(self, name: str):
        return self.probe(name) if self.probe is not None else _NULL

    def _new_buffers(self, s: int, extra: dict | None = None) -> dict:
        d, dev = self.cfg.hidden, self.device
        e = lambda *shape: torch.empty(shape, dtype=torch.bfloat16, device=dev)  # noqa: E731
        bufs = {"h": e(s, d), "n": e(s, d), "qkv": e(s, 3 * d), "ff": e(s, self.cfg.mlp)}
        if self.kind == "fp8":  # LayerNorm output straight to per-token e4m3 + scales
            bufs["nq"] = torch.empty((s, d), dtype=torch.float8_e4m3fn, device=dev)
            bufs["ns"] = torch.empty((s,), dtype=torch.float32, device=dev)
        if self.kind == "mx" and self._ln_mx_fusable():  # LayerNorm output straight to MXFP8
            bufs["nq"] = torch.empty((s, d), dtype=torch.float8_e4m3fn, device=dev)
            bufs["nsx"] = torch.empty((s, d // 32), dtype=torch.uint8, device=dev)
        if self.kind == "mx":  # the MLP hidden activation as MXFP8 codes from FF1's epilogue
            f = self.cfg.mlp
            bufs["ffq"] = torch.empty((s, f), dtype=torch.float8_e4m3fn, device=dev)
            bufs["ffs"] = torch.empty((s, f // 32), dtype=torch.uint8, device=dev)
        for k, shape in (extra or {}).items():
            bufs[k] = e(*shape)
        return bufs

    @staticmethod
    def _mx_mlp(blk) -> None:
        """An MXFP8 MLP pair: FF1's output rows go to swizzle order (FF1 then writes FF2's A
        operand in its epilogue); blk.ff_mx marks the block."""
        pairs = ((blk.ff1_txt, blk.ff2_txt), (blk.ff1_img, blk.ff2_img))
        blk.ff_mx = all(a.kind == "mx" and b.kind == "mx" and a.n % 32 == 0 for a, b in pairs)
        if blk.ff_mx:
            blk.ff1_txt = blk.ff1_txt.rows_in_swizzle_order()
            blk.ff1_img = blk.ff1_img.rows_in_swizzle_order()

    def _ln_mx_fusable(self) -> bool:
        """The LayerNorm -> MXFP8 kernel covers whole 512-wide swizzle tiles."""
        return self.cfg.hidden % 512 == 0

    def _ln(self, bufs, rows: slice, sc, sh, kind: str = "bf16"):
        """adaLN of h[rows] into the next GEMM's A operand, for a GEMM of `kind`: bf16 into n,
        or per-token e4m3 codes and scales (fp8) / swizzled MXFP8 codes and E8M0 scales (mx) in
        one pass. Returns the `prepared` operand (None for bf16)."""
        h = bufs["h"]
        if kind == "fp8" and "ns" in bufs:
            nq, ns = bufs["nq"][rows], bufs["ns"][rows]
            kernels.layernorm_modulate_fp8(h[rows], sc, sh, eps=EPS, out=(nq, ns))
            return nq, ns
        if kind == "mx" and "nsx" in bufs:
            nq, ns = bufs["nq"][rows], bufs["nsx"][rows]
            kernels.layernorm_modulate_mx(h[rows], sc, sh, eps=EPS, out=(nq, ns))
            return nq, ns
        kernels.layernorm_modulate(h[rows], sc, sh, eps=EPS, out=bufs["n"][rows])
        return None

    def _ln_joint(self, bufs, st: int, txt_sc, txt_sh, img_sc, img_sh, kind: str = "bf16"):
        """adaLN of all rows of h in one launch, text rows [0, st) with the text vectors and the
        image rows with the image ones, into the A operands of a GEMM pair of `kind` (as _ln).
        Returns the text and image `prepared` operands."""
        h, s = bufs["h"], bufs["h"].shape[0]
        T, I = slice(0, st), slice(st, s)
        kw = dict(eps=EPS, split=st, mul2=img_sc, add2=img_sh) if st else dict(eps=EPS)
        sc, sh = (txt_sc, txt_sh) if st else (img_sc, img_sh)
        if kind == "fp8" and "ns" in bufs:
            nq, ns = bufs["nq"], bufs["ns"]
            kernels.layernorm_modulate_fp8(h, sc, sh, out=(nq, ns), **kw)
            return (nq[T], ns[T]), (nq[I], ns[I])
        if kind == "mx" and "nsx" in bufs:
            nq, ns = bufs["nq"], bufs["nsx"]
            kernels.layernorm_modulate_mx(h, sc, sh, out=(nq, ns), **kw)
            return (nq[T], ns[T]), (nq[I], ns[I])
        kernels.layernorm_modulate(h, sc, sh, out=bufs["n"], **kw)
        return None, None

    def _prep_joint(self, lin_txt, lin_img, a, st: int, gelu_from: int | None = None):
        """The A operands of a text / image GEMM pair from one activation buffer a [S, K],
        quantized (fp8 kinds) in one launch over all rows (gelu_from: see DeviceLinear.prep)."""
        if lin_txt.kind != lin_img.kind:
            raise ValueError("a joint GEMM pair shares one kind")
        if lin_img.kind == "bf16":
            return None, None
        q, sc = lin_img.prep(a, gelu_from=gelu_from)
        return (q[:st], sc[:st]), (q[st:], sc[st:])

    #: per-token fp8 steps apply the MLP's GELU where its bf16 pre-activation is quantized for
    #: the next GEMM (quantize_fp8_rowwise(gelu_from=...)), not in the producing GEMM's epilogue:
    #: the quantizer is bound by HBM and absorbs the GELU's VALU work, which in a GEMM epilogue
    #: runs while the matrix cores idle
    fp8_gelu_at_quant = True

    def _gelu_at_quant(self, lin) -> bool:
        return lin.kind == "fp8" and self.fp8_gelu_at_quant

    def _attn(self, buf, q_off: int, k_off: int, v_off: int):
        """Joint attention over all rows of `buf` [S, ld]; output written over q."""
        c = self.cfg
        s, ld = buf.shape
        view = lambda off: buf.as_strided((1, c.heads, s, c.head_dim), (0, c.head_dim, ld, 1),  # noqa: E731
                                          buf.storage_offset() + off)
        q, k, v = view(q_off), view(k_off), view(v_off)
        with self._timed("attn"):
            kernels.attention(q, k, v, scale=1.0 / math.sqrt(c.head_dim), out=q)

    def _gemm(self, name: str, problems, kind: str, epilogue: int = 0, act_col_start: int = 0,
              qk=None):
        """One grouped GEMM launch (activation quantization already done by problem())."""
        with self._timed(name):
            run(problems, kind, epilogue, act_col_start, qk)

    def _qk_epilogue(self, q_col, k_col, cos, sin):
        """The fused q/k RMSNorm + RoPE of an attention projection (law 0, per head)."""
        c = self.cfg
        return kernels.QkNormRope(q_col, k_col, c.heads * c.head_dim, cos, sin, law=0, eps=EPS)

    def joint_block(self, blk, bufs, st: int, img_mods, txt_mods, cos, sin, tag: str):
        """One joint block over h (text rows [0, st), image rows [st, S)). blk holds the device
        linears qkv_{txt,img} ([q|k|v] rows), out_{txt,img}, ff1_{txt,img}, ff2_{txt,img} and the
        bf16 RMSNorm weights nq, nk (image) and naq, nak (text)."""
        d = self.cfg.hidden
        h, n, qkv, ff = bufs["h"], bufs["n"], bufs["qkv"], bufs["ff"]
        s = h.shape[0]
        T, I = slice(0, st), slice(st, s)
        x_sh, x_sc, x_g, x_sh2, x_sc2, x_g2 = img_mods
        c_sh, c_sc, c_g, c_sh2, c_sc2, c_g2 = txt_mods
        # every elementwise step runs once over all rows: the text and image rows of each
        # launch differ only in their modulation vectors or norm weights
        pt, pi = self._ln_joint(bufs, st, c_sc, c_sh, x_sc, x_sh, blk.qkv_img.kind)
        # q/k RMSNorm (text rows with the added-stream weights) and RoPE in the GEMM epilogue
        self._gemm(f"gemm.{tag}.qkv",
                   [blk.qkv_txt.problem(n[T], qkv[T], prepared=pt, norm_q=blk.naq,
                                        norm_k=blk.nak, rope_row0=0),
                    blk.qkv_img.problem(n[I], qkv[I], prepared=pi, norm_q=blk.nq,
                                        norm_k=blk.nk, rope_row0=st)],
                   blk.qkv_img.kind, qk=self._qk_epilogue(0, d, cos, sin))
        self._attn(qkv, 0, d, 2 * d)
        o = qkv[:, :d]
        pt, pi = self._prep_joint(blk.out_txt, blk.out_img, o, st)
        self._gemm(f"gemm.{tag}.out",
                   [blk.out_txt.problem(o[T], h[T], gate=c_g, residual=h[T], prepared=pt),
                    blk.out_img.problem(o[I], h[I], gate=x_g, residual=h[I], prepared=pi)],
                   blk.out_img.kind, _lib.EPI_GATE_RESIDUAL)
        pt, pi = self._ln_joint(bufs, st, c_sc2, c_sh2, x_sc2, x_sh2, blk.ff1_img.kind)
        if getattr(blk, "ff_mx", False) and "ffq" in bufs:
            # FF1's epilogue writes GELU(x) as MXFP8 codes and scales, FF2's A operand: FF1's
            # weight rows are in swizzle order, so its output columns are FF2's swizzled K
            fq, fs = bufs["ffq"], bufs["ffs"]
            self._gemm(f"gemm.{tag}.ff1",
                       [blk.ff1_txt.problem(n[T], fq[T], prepared=pt, c_scale=fs[T]),
                        blk.ff1_img.problem(n[I], fq[I], prepared=pi, c_scale=fs[I])],
                       "mx", _lib.EPI_GELU_MX)
            pt, pi = (fq[T], fs[T]), (fq[I], fs[I])
        else:
            late = self._gelu_at_quant(blk.ff2_img)  # fp8: FF1 stores the pre-activation
            self._gemm(f"gemm.{tag}.ff1", [blk.ff1_txt.problem(n[T], ff[T], prepared=pt),
                                           blk.ff1_img.problem(n[I], ff[I], prepared=pi)],
                       blk.ff1_img.kind, _lib.EPI_NONE if late else _lib.EPI_GELU)
            pt, pi = self._prep_joint(blk.ff2_txt, blk.ff2_img, ff, st,
                                      gelu_from=0 if late else None)
        self._gemm(f"gemm.{tag}.ff2",
                   [blk.ff2_txt.problem(ff[T], h[T], gate=c_g2, residual=h[T], prepared=pt),
                    blk.ff2_img.problem(ff[I], h[I], gate=x_g2, residual=h[I], prepared=pi)],
                   blk.ff2_img.kind, _lib.EPI_GATE_RESIDUAL)
