"""Builds libpagellm_hip.so in-tree with hipcc for gfx950.

    python -m pagellm_amd.build [--verbose]

The library is placed next to this file so the ctypes loader (and a copy of
the tree on another machine) finds it without installation.
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libpagellm_hip.so"
BUILD = PKG / "_build"
SOURCES = ["plh_sample.hip", "plh_verify.hip", "plh_head.hip", "plh_api.hip"]
HEADERS = ["plh_device.h", "plh_pipeline.h", "plh_kernels.h"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("PLH_OFFLOAD_ARCH", "gfx950")
# IEEE float64 division and exp are part of the contract: no fast-math.
# Packed FP32 instructions are disabled for every kernel.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ... (exit {r.returncode})")
    if verbose and (r.stdout or r.stderr):
        sys.stderr.write(r.stdout + r.stderr)


STAMPS_DIR = PKG / "_stamps"  # the profiling build (--phase-stamps)


def build(verbose: bool = False, extra: list[str] | None = None, phase_stamps: bool = False) -> Path:
    """Compile every HIP source and link the shared library.  Always
    recompiles (a stale library must never hide a source change).  With
    phase_stamps, a profiling build that records k_sample_final's phase
    clock stamps (-DPLH_PHASE_STAMPS) goes to _stamps/ instead."""
    build_dir = STAMPS_DIR / "_build" if phase_stamps else BUILD
    out = STAMPS_DIR / OUT.name if phase_stamps else OUT
    build_dir.mkdir(parents=True, exist_ok=True)
    extra = list(extra or []) + (["-DPLH_PHASE_STAMPS"] if phase_stamps else [])
    include = ["-I", str(CSRC), "-I", str(PKG.parent / "include")]

    def compile_one(src: str) -> Path:
        obj = build_dir / (Path(src).stem + ".o")
        _run([HIPCC, *FLAGS, *extra, *include, "-c", str(CSRC / src), "-o", str(obj)], verbose)
        return obj

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, *FLAGS, "-shared", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, out)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--resource-usage", action="store_true", help="print per-kernel register/LDS usage")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="profiling build with k_sample_final's phase clock stamps, to pagellm_amd/_stamps/")
    args = ap.parse_args()
    extra = ["-Rpass-analysis=kernel-resource-usage"] if args.resource_usage else []
    print(build(verbose=args.verbose or args.resource_usage, extra=extra, phase_stamps=args.phase_stamps))


if __name__ == "__main__":
    main()
