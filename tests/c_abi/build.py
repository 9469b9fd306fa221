"""Builds tests/c_abi/fagq_c_check, a plain C host program that calls
libfagq.so through include/fagq.h (gcc, linked against the in-tree library
and the HIP runtime; the rpath points at both, so it runs from the tree)."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
PKG_DIR = REPO / "flagos-kernelgen-72h-shanghai-2026_amd"
EXE = HERE / "fagq_c_check"


def build() -> Path:
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    cmd = ["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
           f"-I{rocm / 'include'}", f"-I{REPO / 'include'}", str(HERE / "fagq_c_check.c"),
           f"-L{PKG_DIR}", "-lfagq", f"-L{rocm / 'lib'}", "-lamdhip64",
           f"-Wl,-rpath,{PKG_DIR}:{rocm / 'lib'}", "-o", str(EXE)]
    subprocess.run(cmd, check=True)
    return EXE


if __name__ == "__main__":
    print(build())
