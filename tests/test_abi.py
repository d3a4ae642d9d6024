"""The C ABI library loads on the CPU host and exports every symbol include/difflet_rocm.h
declares (no compute calls: there is no GPU here)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "difflet_rocm.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(difflet_rocm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_python_signatures():
    from difflet_amd import _lib

    assert declared_symbols() == _lib.exported_symbols()


def test_library_loads_and_exports_every_declared_symbol():
    from difflet_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (python -m difflet_amd.csrc.build)")
    lib = _lib.load()
    for name in declared_symbols():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name
    assert lib.difflet_rocm_abi_version() == 1
    assert b"gfx950" in lib.difflet_rocm_version()


def test_error_paths_report_without_a_gpu():
    """Argument validation runs before any device call, so bad calls fail cleanly here."""
    from difflet_amd import _lib

    lib = _lib.load()
    st = lib.difflet_rocm_gemm_bf16(0, None, 64, 64, 0, 0, None)
    assert st == _lib.EINVAL
    assert b"nproblems" in lib.difflet_rocm_last_error()
    st = lib.difflet_rocm_attention(None, None, None, None, _lib.BF16, 1, 1, 1, 1, 128, None,
                                    None, None, None, 1.0, 0, None, 0, None, None, None, None,
                                    None)
    assert st == _lib.EINVAL
    with pytest.raises(ValueError):
        _lib.check(st, "attention")
