"""Loads libdifflet_rocm.so (the C ABI in include/difflet_rocm.h) and declares its signatures.

The library is built in place by ``python -m difflet_amd.csrc.build`` (or
``__graft_entry__.build()``). There is no fallback: if the library is missing or cannot be
loaded, every op of the rocm backend raises instead of silently running something else.

torch is imported first on purpose: PyTorch-ROCm ships its own HIP runtime, and the library
must bind to that same runtime instance (same SONAME) so torch's device pointers and streams
are valid in it.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (see module docstring: binds the HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / "libdifflet_rocm.so"

# enum difflet_dtype
F32, BF16, F16, U8, BOOL, I32 = 0, 1, 2, 3, 4, 5
# enum difflet_status
OK, EINVAL, EUNSUPPORTED, ELAUNCH = 0, 1, 2, 3
# enum difflet_epilogue
EPI_NONE, EPI_GELU, EPI_GATE_RESIDUAL, EPI_GELU_MX, EPI_F32 = 0, 1, 2, 3, 4

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_i64p = ctypes.POINTER(ctypes.c_int64)


class GemmProblem(ctypes.Structure):
    """``difflet_gemm_problem`` of include/difflet_rocm.h."""

    _fields_ = [
        ("a", _vp), ("lda", _i64),
        ("w", _vp), ("ldw", _i64),
        ("c", _vp), ("ldc", _i64),
        ("bias", _vp),
        ("gate", _vp), ("gate_stride", _i64),
        ("residual", _vp), ("ldr", _i64),
        ("a_scale", _vp), ("w_scale", _vp),
        ("m", _i64), ("rows_per_batch", _i64),
        ("norm_q", _vp), ("norm_k", _vp), ("rope_row0", _i64),
        ("c_scale", _vp), ("ld_c_scale", _i64),
    ]


class GemmQk(ctypes.Structure):
    """``difflet_gemm_qk`` of include/difflet_rocm.h."""

    _fields_ = [
        ("q_col", _i64), ("k_col", _i64), ("cols", _i64),
        ("cos", _vp), ("sin", _vp),
        ("law", _i32), ("eps", _f32), ("rows", _i64),
    ]


#: name -> (restype, argtypes); the declarations of include/difflet_rocm.h.
SIGNATURES: dict[str, tuple] = {
    "difflet_rocm_last_error": (ctypes.c_char_p, []),
    "difflet_rocm_version": (ctypes.c_char_p, []),
    "difflet_rocm_abi_version": (_i32, []),
    "difflet_rocm_device_count": (_i32, []),
    "difflet_rocm_attention": (_i32, [
        _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64,
        _i64p, _i64p, _i64p, _i64p, _f32, _i32, _vp, _i32, _i64p, _vp, _vp, _i64p, _vp, _i64,
        _vp]),
    "difflet_rocm_attention_workspace_bytes": (_i64, []),
    "difflet_rocm_attention_noalloc": (_i32, [
        _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64,
        _i64p, _i64p, _i64p, _i64p, _f32, _i32, _vp, _i32, _i64p, _vp, _vp, _i64p, _vp]),
    "difflet_rocm_gemm_workspace_bytes": (_i64, []),
    "difflet_rocm_gemm_bf16": (_i32, [_i32, ctypes.POINTER(GemmProblem), _i64, _i64, _i32,
                                      _i64, _vp, _i64, ctypes.POINTER(GemmQk), _vp]),
    "difflet_rocm_gemm_fp8_rowwise": (_i32, [_i32, ctypes.POINTER(GemmProblem), _i64, _i64,
                                             _i32, _i64, _vp, _i64, ctypes.POINTER(GemmQk), _vp]),
    "difflet_rocm_gemm_mxfp8": (_i32, [_i32, ctypes.POINTER(GemmProblem), _i64, _i64, _i32,
                                       _i64, _vp, _i64, ctypes.POINTER(GemmQk), _vp]),
    "difflet_rocm_gemm_schedule_check": (_i32, [_i32, _i32, _i32, _i32, _i64,
                                                ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "difflet_rocm_attention_schedule_check": (_i32, [_i64, _i32, _i32, _i64,
                                                     ctypes.POINTER(_i32),
                                                     ctypes.POINTER(_i32)]),
    "difflet_rocm_quantize_fp8_rowwise": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp,
                                                 _vp]),
    "difflet_rocm_quantize_fp8_rowwise_gelu": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64,
                                                      _vp, _i64, _vp]),
    "difflet_rocm_quantize_mxfp8": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _i64,
                                           _i32, _vp]),
    "difflet_rocm_layernorm_modulate": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _i64, _i64,
                                               _vp, _vp, _i32, _i64, _i64, _i64, _i32, _f32,
                                               _vp]),
    "difflet_rocm_layernorm_modulate_fp8": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _i64, _i64,
                                                   _vp, _vp, _i32, _i64, _i64, _i64, _i32, _f32,
                                                   _vp]),
    "difflet_rocm_layernorm_modulate_mx": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _i64,
                                                  _i64, _vp, _vp, _i32, _i64, _i64, _i64, _i32,
                                                  _f32, _vp]),
    "difflet_rocm_rms_norm": (_i32, [_vp, _i64, _vp, _i64, _i32, _i64, _i64, _vp, _i32, _f32,
                                     _vp]),
    "difflet_rocm_qk_norm_rope": (_i32, [_vp, _i64, _i32, _i64, _i64, _i64, _i64, _i64, _i32,
                                         _vp, _vp, _i64, _vp, _vp, _i32, _f32, _vp, _vp, _i64,
                                         _i32, _vp]),
    "difflet_rocm_rope": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                 _vp, _vp, _i64, _i32, _vp]),
    "difflet_rocm_gelu_tanh": (_i32, [_vp, _vp, _i32, _i64, _vp]),
    "difflet_rocm_gate_residual": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i64, _i64, _i64,
                                          _i64, _vp]),
    "difflet_rocm_gemv": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                                 _i32, _vp]),
    "difflet_rocm_timestep_embedding": (_i32, [_vp, _vp, _i32, _i64, _i64, _i32, _f32, _f32,
                                               _f32, _vp]),
    "difflet_rocm_gemm_f32": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64,
                                     _i64, _i64, _vp]),
    "difflet_rocm_gated_gelu": (_i32, [_vp, _i64, _vp, _i64, _i32, _i64, _i64, _vp]),
    "difflet_rocm_embedding": (_i32, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp]),
    "difflet_rocm_relative_bias": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i64, _i64, _vp,
                                          _i64, _vp, _vp]),
    "difflet_rocm_group_norm_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "difflet_rocm_group_norm": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _f32,
                                       _i32, _vp, _i64, _vp]),
    "difflet_rocm_im2col3x3": (_i32, [_vp, _i32, _i64, _i64, _i64, _i32, _i64, _i64, _vp, _i64,
                                      _i64, _vp]),
    "difflet_rocm_softmax_rows": (_i32, [_vp, _i64, _vp, _i64, _i32, _i64, _i64, _f32, _vp]),
    "difflet_rocm_im2col_causal": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _i32, _i64, _i64,
                                          _i64, _i64, _i64, _i32, _i64, _i64, _vp, _i64, _i64,
                                          _vp]),
    "difflet_rocm_conv_causal": (_i32, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64,
                                        _i64, _i64, _i64, _i64, _i32, _i64, _vp, _i64, _i64, _vp,
                                        _vp, _i64, _vp, _i64, _vp, _i64, _vp]),
    "difflet_rocm_conv_causal_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "difflet_rocm_rms_norm_channels": (_i32, [_vp, _i64, _vp, _i64, _i32, _i64, _i64, _vp, _f32,
                                              _i32, _vp]),
    "difflet_rocm_rows_to_planes": (_i32, [_vp, _i64, _i32, _i64, _i64, _vp, _f32, _f32, _vp]),
}

_lib = None
_lock = threading.Lock()


class LibraryNotBuilt(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """The loaded library with every signature declared; raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise LibraryNotBuilt(
                f"{p} is missing: build the HIP kernels first "
                "(python -m difflet_amd.csrc.build)")
        lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Raises the Python exception matching a difflet_status."""
    if status == OK:
        return
    msg = load().difflet_rocm_last_error().decode(errors="replace")
    if status == EINVAL:
        raise ValueError(f"{what}: {msg}")
    if status == EUNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {status})")


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)
