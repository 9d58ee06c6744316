"""Build libflash_mlm_hip.so for gfx950 from csrc/*.hip with hipcc.

Usage: python flash-mlm_amd/build_lib.py [--jobs N] [--verbose]

Objects go to flash-mlm_amd/_build/, the shared library to
flash-mlm_amd/flash_mlm/_native/libflash_mlm_hip.so (both git-ignored; the
library travels with the source tree to the GPU host).
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
BUILD = PKG_ROOT / "_build"
OUT_DIR = PKG_ROOT / "flash_mlm" / "_native"
LIB_NAME = "libflash_mlm_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-but-set-variable",
    # no packed fp32 instructions in device code (wrong results seen on this pool)
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    if not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources under csrc/")
    objs = []
    cmds = []
    for src in sources:
        obj = BUILD / (src.stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)])
    jobs = jobs or min(len(cmds), os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    _run(
        [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)],
        verbose,
    )
    final = OUT_DIR / LIB_NAME
    os.replace(tmp, final)
    return final


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--clean", action="store_true")
    args = ap.parse_args()
    if args.clean and BUILD.exists():
        shutil.rmtree(BUILD)
    path = build(args.jobs, args.verbose)
    print(path)


if __name__ == "__main__":
    main()
