"""Build libmixmoe.so (gfx950) in-tree with hipcc (linked against the HIP
runtime only).

Every HIP source is compiled with -ffp-contract=off (the routing arithmetic
must match the CPU restatement operation for operation) and with packed-fp32
instruction selection disabled.  Objects go to mixlab_amd/_build/, the shared
library to mixlab_amd/libmixmoe.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libmixmoe.so"
SOURCES = [
    "mxm_router.hip",
    "mxm_dispatch.hip",
    "mxm_gemm_simt.hip",
    "mxm_gemm_mfma.hip",
    "mxm_wgrad.hip",
    "mxm_decode.hip",
    "mxm_prep.hip",
    "mxm_block.hip",
    "mxm_backward.hip",
    "mxm_abi.hip",
]
ARCH = os.environ.get("MIXMOE_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-mllvm", "-disable-promote-alloca-to-lds",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-Wno-inline-asm",  # the direct-to-LDS load names M0 in its clobber list
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: libmixmoe needs ROCm's hipcc to build")


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link libmixmoe.so; returns the library path."""
    BUILD.mkdir(exist_ok=True)
    objs = [BUILD / (Path(s).stem + ".o") for s in SOURCES]
    jobs = min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _compile(CSRC / so[0], so[1]), zip(SOURCES, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
