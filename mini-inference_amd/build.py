"""Build libmipaged.so (the C-ABI HIP library) in-tree for gfx950.

Usage: python mini-inference_amd/build.py [--jobs N] [--verbose]

Every ``csrc/*.hip`` file is compiled to an object in ``_build/`` (in parallel), then the
objects are linked into ``engine/libmipaged.so`` next to the Python package that loads it.
The library always targets gfx950 only.
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
LIB = PKG_ROOT / "engine" / "libmipaged.so"
INCLUDE = PKG_ROOT.parent / "include"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU ops (v_pk_fma_f32 and friends) stay disabled for every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs (the softmax rescale and the epilogue work on them with VALU
    # ops; AGPR placement costs a copy each way per tile).
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
]
# Per-source flags. The stream decode kernels take their plan pointer and word offsets as
# leading scalar arguments; preloading them into scalar registers at wave launch (gfx950
# kernel-argument preloading) lets a kernel's first plan reads go out without waiting for a
# load of its arguments. Code objects keep a fallback that loads them where the firmware does
# not preload.
FILE_FLAGS = {
    "paged_decode_stream.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=3"],
    # The read probe (the ceiling the decode kernel is compared with) launches the same way.
    "hbm_probe.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=3"],
    # The KV append takes its slot list and source rows as leading arguments in the same way.
    "kv_append.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=3"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmipaged.so)")


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag; that warning is noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), sources))
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
