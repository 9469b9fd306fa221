"""Builds the C oracle (test infrastructure) into oracle/libfagq_oracle.so:
fagq_oracle.c (the operator), gemm_oracle.c (the fp8 block-scaled GEMM that
consumes the operator's output) and dsa_topk_oracle.c (the Task 02 DSA top-k
page-table transform).

The oracle restates the reference's algorithm on the CPU and is used only as
the checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg.  The reference repository itself is Python/Triton: there is no native
reference source to compile, so there is no oracle/_ref build.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SRCS = [ORACLE_DIR / "fagq_oracle.c", ORACLE_DIR / "gemm_oracle.c", ORACLE_DIR / "dsa_topk_oracle.c",
        ORACLE_DIR / "mla_bwd_oracle.c"]
LIB = ORACLE_DIR / "libfagq_oracle.so"

CFLAGS = ["-O2", "-std=gnu11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-fno-fast-math", "-fvisibility=hidden", "-Wall", "-Wextra"]


def build(verbose: bool = False) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", *CFLAGS, "-o", str(tmp), *[str(s) for s in SRCS], "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}")
    if verbose and res.stdout.strip():
        print(res.stdout, flush=True)
    os.replace(tmp, LIB)
    return LIB


def build_sanitized(verbose: bool = False) -> Path:
    """The same sources built with clang's AddressSanitizer and
    UndefinedBehaviorSanitizer into oracle/_build_san/libfagq_oracle.so, for the
    CPU tests' sanitizer run (which preloads clang's shared ASan runtime, the
    one the product library's sanitizer build uses too)."""
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    clang = rocm / "llvm" / "bin" / "clang"
    out_dir = ORACLE_DIR / "_build_san"
    out_dir.mkdir(exist_ok=True)
    out = out_dir / "libfagq_oracle.so"
    cflags = [f for f in CFLAGS if f != "-O2"] + ["-O1", "-g", "-fno-omit-frame-pointer",
                                                  "-fsanitize=address,undefined",
                                                  "-fno-sanitize-recover=undefined", "-shared-libsan"]
    cmd = [str(clang), *cflags, "-o", str(out), *[str(s) for s in SRCS], "-lm",
           f"-Wl,-rpath,{rocm / 'llvm' / 'lib'}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"sanitized oracle build failed:\n{res.stdout}")
    return out


if __name__ == "__main__":
    print(build(verbose=True))
