"""Build libmoddit.so (the gfx950 C-ABI library) in-tree with hipcc.

Every HIP source under csrc/ is compiled for gfx950 in parallel and linked into one
shared library next to this file. No CUDA headers, no dual paths: the sources are
HIP/CDNA4 only.

    python mod-dit_amd/build.py            # build
    python mod-dit_amd/build.py --verbose  # echo commands
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libmoddit.so"
LIB_PATH = PKG_DIR / LIB_NAME
# measurement aids (MFMA ceiling on random operands for bench.py, single-MFMA accumulation
# precision for the int8/fp8 accuracy contract); not part of the C ABI
CALIB_SRCS = (CSRC / "calib" / "mfma_ceiling.hip", CSRC / "calib" / "mfma_precision.hip")
CALIB_PATH = PKG_DIR / "libmoddit_calib.so"

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # Packed fp32 VALU forms are kept out of every kernel (they have given wrong
    # results on these boxes); the host pass warns that it does not know the feature.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build libmoddit.so)")
    return path


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile csrc/*.hip for gfx950 and link libmoddit.so (and the calibration library);
    returns the path of libmoddit.so."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in sources:
        obj = BUILD_DIR / (src.stem + ".o")
        objs.append(obj)
        cmds.append([cc, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)])
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB_PATH)
    build_calib(verbose)
    return LIB_PATH


def build_calib(verbose: bool = False) -> Path:
    """Compile the MFMA measurement kernels into libmoddit_calib.so."""
    tmp = CALIB_PATH.with_suffix(".so.tmp")
    _run([hipcc(), *COMMON_FLAGS, "-shared", "-o", str(tmp), *map(str, CALIB_SRCS)], verbose)
    os.replace(tmp, CALIB_PATH)
    return CALIB_PATH


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    args = ap.parse_args(argv)
    path = build_library(verbose=args.verbose, jobs=args.jobs)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
