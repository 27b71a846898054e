"""Compile the C11 caller of libmixmoe (known_answer.c) with gcc against
include/mixmoe.h and mixlab_amd/libmixmoe.so.  The binary goes to
tests/c_abi/_build/known_answer, with an rpath to the library's directory,
so it runs from any working directory."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
SRC = HERE / "known_answer.c"
OUT = HERE / "_build" / "known_answer"
FLAGS = ["-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-pedantic"]


def compile_caller(out: Path = OUT) -> Path:
    lib_dir = ROOT / "mixlab_amd"
    if not (lib_dir / "libmixmoe.so").exists():
        raise RuntimeError("mixlab_amd/libmixmoe.so is missing: build the library first")
    out.parent.mkdir(parents=True, exist_ok=True)
    rel = os.path.relpath(lib_dir, out.parent)
    cmd = ["gcc", *FLAGS, f"-I{ROOT / 'include'}", str(SRC), "-o", str(out), f"-L{lib_dir}",
           "-lmixmoe", f"-Wl,-rpath,$ORIGIN/{rel}", "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed:\n{' '.join(cmd)}\n{res.stderr}")
    return out


if __name__ == "__main__":
    print(compile_caller(Path(sys.argv[1]) if len(sys.argv) > 1 else OUT))
