"""Build libgeoweave_hip.so (gfx950) in-tree with hipcc.

    python -m geoweave_amd.build [-v]

Every ``csrc/*.hip`` file is compiled to an object in ``geoweave_amd/_build/`` (in
parallel) and linked into ``geoweave_amd/libgeoweave_hip.so``. The flags target gfx950
only and disable packed-fp32 instruction selection.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libgeoweave_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO_DIR / 'include'}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the gfx950 library needs the ROCm toolchain")


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    res = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag; that warning is noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(map(str, cmd))}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objects = [BUILD_DIR / (s.stem + ".o") for s in sources]

    def compile_one(pair):
        src, obj = pair
        _run([hipcc, *COMMON_FLAGS, "-c", src, "-o", obj], verbose)

    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(sources)))) as ex:
        list(ex.map(compile_one, zip(sources, objects)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", tmp], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=8)
    args = ap.parse_args()
    path = build(verbose=args.verbose, jobs=args.jobs)
    print(path)


if __name__ == "__main__":
    main()
