"""Builds libdifflet_rocm.so for gfx950 in place (next to the difflet_amd package).

Each .hip source compiles to its own object in parallel, then one link. hipcc cross-compiles
without a GPU, so this runs on any host with ROCm installed.

    python -m difflet_amd.csrc.build [--jobs N] [--verbose]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
REPO = PKG.parent
LIB_NAME = "libdifflet_rocm.so"
LIB_PATH = PKG / LIB_NAME
OBJ_DIR = REPO / "_build" / "difflet_rocm"
SOURCES = ("runtime.hip", "elementwise.hip", "gemm.hip", "gemm_f32.hip", "attention.hip",
           "quant.hip", "vae.hip", "conv.hip")
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc must not form v_pk_{add,mul,fma}_f32 on its own.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(REPO / "include"),
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build the kernels")
    return path


def _compile(src: Path, obj: Path, verbose: bool) -> tuple[Path, str]:
    cmd = [hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops" not in line  # the host pass does not know the feature: harmless
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{log}")
    return obj, log


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, CSRC / s, OBJ_DIR / (Path(s).stem + ".o"), verbose)
                for s in SOURCES]
        for f in futs:
            obj, log = f.result()
            if log.strip() and verbose:
                print(log)
            objs.append(obj)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(args.jobs, args.verbose)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
