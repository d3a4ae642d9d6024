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
    assert lib.difflet_rocm_abi_version() == 7
    assert b"gfx950" in lib.difflet_rocm_version()


def test_error_paths_report_without_a_gpu():
    """Argument validation runs before any device call, so bad calls fail cleanly here."""
    from difflet_amd import _lib

    lib = _lib.load()
    st = lib.difflet_rocm_gemm_bf16(0, None, 64, 64, 0, 0, None, 0, None, None)
    assert st == _lib.EINVAL
    assert b"nproblems" in lib.difflet_rocm_last_error()
    st = lib.difflet_rocm_attention(None, None, None, None, _lib.BF16, 1, 1, 1, 1, 128, None,
                                    None, None, None, 1.0, 0, None, 0, None, None, None, None,
                                    None, 0, None)
    assert st == _lib.EINVAL
    with pytest.raises(ValueError):
        _lib.check(st, "attention")


@pytest.mark.parametrize("cus", [256, 304, 80])
def test_gemm_split_schedule_covers_every_stage_once(cus):
    """The GEMMs' split schedule, walked on the host with the kernels' own functions: every
    (tile, K stage) runs exactly once, cut tiles are summed from their true contributors, and
    no two cut tiles share a workspace slot."""
    import ctypes

    from difflet_amd import _lib

    lib = _lib.load()
    ws = 16384 + 2 * cus * 256 * 256 * 4
    dp, groups = ctypes.c_int(), ctypes.c_int()
    split = 0
    for tiles in list(range(1, 40)) + [216, 255, 256, 257, 336, 392, 648, 864, 1008, 1344,
                                       1512, 7 * cus + 5]:
        for nk, gran in ((1, 1), (2, 1), (7, 1), (8, 1), (48, 1), (96, 1), (192, 1), (480, 1),
                         (6, 4), (48, 4), (50, 4), (192, 4), (48, 8)):
            r = lib.difflet_rocm_gemm_schedule_check(tiles, nk, gran, cus, ws, ctypes.byref(dp),
                                                     ctypes.byref(groups))
            assert r == 0, (tiles, nk, gran, r)
            assert 0 <= dp.value <= tiles
            if groups.value:
                split += 1
                assert dp.value % cus == 0 and groups.value <= cus
    assert split > 50  # the split path is exercised


def test_gemm_split_plan_at_the_step_shapes():
    import ctypes

    from difflet_amd import _lib

    lib = _lib.load()
    ws = 16384 + 2 * 256 * 256 * 256 * 4
    dp, groups = ctypes.c_int(), ctypes.c_int()
    # Qwen-Image's 336-tile launches run a wave of whole tiles and cut the last 80 over the
    # 256 CUs; FLUX's 216-tile ones (the cut would save an eighth) and a 1512-tile one (98 %
    # full) stay whole
    assert lib.difflet_rocm_gemm_schedule_check(336, 48, 1, 256, ws, ctypes.byref(dp),
                                                ctypes.byref(groups)) == 0
    assert (dp.value, groups.value) == (256, 256)
    assert lib.difflet_rocm_gemm_schedule_check(336, 192, 8, 256, ws, ctypes.byref(dp),
                                                ctypes.byref(groups)) == 0
    assert (dp.value, groups.value) == (256, 256)
    assert lib.difflet_rocm_gemm_schedule_check(216, 96, 1, 256, ws, ctypes.byref(dp),
                                                ctypes.byref(groups)) == 0
    assert (dp.value, groups.value) == (216, 0)
    assert lib.difflet_rocm_gemm_schedule_check(1512, 96, 1, 256, ws, ctypes.byref(dp),
                                                ctypes.byref(groups)) == 0
    assert (dp.value, groups.value) == (1512, 0)
    # MXFP8 (units of 4 K stages of 128) with a shorter last unit: K = 6912 (54 stages, the last
    # unit 2) at Qwen-Image's 336 tiles, K = 7808 (61 stages, the last unit 1) on 15 tiles;
    # both split, as the device tests of these shapes assume
    assert lib.difflet_rocm_gemm_schedule_check(336, 54, 4, 256, ws, ctypes.byref(dp),
                                                ctypes.byref(groups)) == 0
    assert (dp.value, groups.value) == (256, 256)
    assert lib.difflet_rocm_gemm_schedule_check(15, 61, 4, 256, ws, ctypes.byref(dp),
                                                ctypes.byref(groups)) == 0
    assert (dp.value, groups.value) == (0, 256)
    # a cut that saves under 24 K stages stays whole: Wan's 80-tile text k/v projection
    # (K = 4096) splits in bf16 (64 stages, 24 per XCD) but not in MXFP8 (8 units of 4, 3 per
    # XCD: 20 stages saved), nor do fp8 and MXFP8 at 336 tiles and K = 3072
    for nk, gran, plan in ((64, 1, (0, 256)), (8, 4, (80, 0))):
        assert lib.difflet_rocm_gemm_schedule_check(80, nk, gran, 256, ws, ctypes.byref(dp),
                                                    ctypes.byref(groups)) == 0
        assert (dp.value, groups.value) == plan
    for nk, gran in ((24, 1), (24, 4)):
        assert lib.difflet_rocm_gemm_schedule_check(336, nk, gran, 256, ws, ctypes.byref(dp),
                                                    ctypes.byref(groups)) == 0
        assert (dp.value, groups.value) == (336, 0)
    # without enough workspace nothing is split
    assert lib.difflet_rocm_gemm_schedule_check(336, 48, 1, 256, 1 << 20, ctypes.byref(dp),
                                                ctypes.byref(groups)) == 0
    assert (dp.value, groups.value) == (336, 0)


@pytest.mark.parametrize("cus", [256, 304, 80, 32])
def test_attention_split_schedule_covers_every_unit_once(cus):
    """The attention's split schedule (whole rounds, then lockstep sets over the cut tiles),
    walked on the host with the kernel's own functions: every (query tile, key tile) runs
    exactly once, a cut tile is merged from the sets that hold its key tiles, and no two parts
    share a workspace slot."""
    import ctypes

    from difflet_amd import _lib

    lib = _lib.load()
    ws = 16384 + 2 * cus * (8 * 16 * 1024 + 8 * 64 * 8)
    dp, w = ctypes.c_int(), ctypes.c_int()
    split = 0
    for tiles in list(range(1, 12)) + [cus - 1, cus, cus + 1, cus + 7, 2 * cus - 3, 432, 672,
                                       1000, 5120, 7 * cus + 5]:
        for key_tiles in (1, 2, 3, 17, 64, 72, 112, 512):
            r = lib.difflet_rocm_attention_schedule_check(tiles, key_tiles, cus, ws,
                                                          ctypes.byref(dp), ctypes.byref(w))
            assert r == 0, (tiles, key_tiles, r)
            if w.value:
                split += 1
                assert dp.value % cus == 0 and 0 < tiles - dp.value < cus
                assert (cus // 8) % w.value == 0
            else:
                assert dp.value == 0
    assert split > 20  # the split path is exercised


def test_attention_split_plan_at_the_step_shapes():
    import ctypes

    from difflet_amd import _lib

    lib = _lib.load()
    ws = 16384 + 2 * 256 * (8 * 16 * 1024 + 8 * 64 * 8)
    dp, w = ctypes.c_int(), ctypes.c_int()
    # FLUX 24 heads x 18 query tiles, 72 key tiles: a round of 256 whole tiles, then 176 cut
    # over 16 sets of 16 (11 groups: 49.5 key tiles per set; sets of 32 would take 54)
    assert lib.difflet_rocm_attention_schedule_check(432, 72, 256, ws, ctypes.byref(dp),
                                                     ctypes.byref(w)) == 0
    assert (dp.value, w.value) == (256, 16)
    # Qwen-Image 24 x 28 query tiles, 112 key tiles: 160 cut tiles in 5 groups of 32
    assert lib.difflet_rocm_attention_schedule_check(672, 112, 256, ws, ctypes.byref(dp),
                                                     ctypes.byref(w)) == 0
    assert (dp.value, w.value) == (512, 32)
    # Wan 40 x 128 query tiles fill 20 rounds exactly: no split; nor without the workspace
    assert lib.difflet_rocm_attention_schedule_check(5120, 512, 256, ws, ctypes.byref(dp),
                                                     ctypes.byref(w)) == 0
    assert (dp.value, w.value) == (0, 0)
    assert lib.difflet_rocm_attention_schedule_check(432, 72, 256, 1 << 20, ctypes.byref(dp),
                                                     ctypes.byref(w)) == 0
    assert (dp.value, w.value) == (0, 0)
