"""Builds libfagq.so, the gfx950 HIP library behind the operators, and
libfagq_probe.so, the measurement probes (HBM streams, matrix-instruction
rate, LDS reads) that are not part of the drop-in library.

Every HIP translation unit is compiled by hipcc for gfx950 only, in
parallel, into ``_build/``; the objects are linked into the two libraries
next to this file, which is what the Python layer loads.  Runs on a machine
without a GPU (hipcc cross-compiles).
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
OBJ_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libfagq.so"
PROBE_LIB_PATH = PKG_DIR / "libfagq_probe.so"
LIB_UNITS = ("fagq_api", "fagq_device", "fagq_gemm", "dsa_topk", "mla_bwd")
PROBE_UNITS = ("fagq_probe", "fagq_device")

ARCH = "gfx950"
# (code format, scale format) pairs compiled from fagq_inst.hip:
# code 0 = fp8 e4m3fn, 1 = int8 round-half-even, 2 = int8 truncate;
# scale 0 = fp32, 1 = ue8m0.
INST_COMBOS = [(q, s) for q in (0, 1, 2) for s in (0, 1)]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def device_flags() -> list[str]:
    # Packed-fp32 instructions are disabled on purpose: the kernels are written
    # with scalar fp32 arithmetic and must not be auto-vectorised into them.
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-fvisibility=hidden",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "-packed-fp32-ops' is not a recognized feature"
    lines = [l for l in res.stdout.splitlines() if noise not in l and l.strip()]
    if verbose and lines:
        print("\n".join(lines), flush=True)


def pyext_path() -> Path:
    import sysconfig
    return PKG_DIR / ("_fagq_py" + sysconfig.get_config_var("EXT_SUFFIX"))


def pyext_command() -> list[str]:
    """g++ line of the CPython binding (csrc/fagq_py.cpp) against torch's headers.
    Host code only: it calls fagq_launch through a pointer it is handed at import."""
    import sysconfig
    import torch
    from torch.utils import cpp_extension
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    return ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            *[f"-I{p}" for p in cpp_extension.include_paths()],
            f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
            str(CSRC / "fagq_py.cpp"), "-o", str(pyext_path().with_suffix(".so.tmp")),
            *[f"-L{p}" for p in cpp_extension.library_paths()],
            "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles every HIP unit for gfx950 and links libfagq.so (and the CPython
    binding of the operator's per-call path); returns the library's path."""
    OBJ_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    flags = device_flags()
    units: list[tuple[Path, Path, list[str]]] = []
    for q, s in INST_COMBOS:
        units.append((CSRC / "fagq_inst.hip", OBJ_DIR / f"fagq_inst_q{q}_s{s}.o",
                      [f"-DFAGQ_QF={q}", f"-DFAGQ_SF={s}"]))
        units.append((CSRC / "fagq_inst_typed.hip", OBJ_DIR / f"fagq_inst_typed_q{q}_s{s}.o",
                      [f"-DFAGQ_QF={q}", f"-DFAGQ_SF={s}"]))
    for unit in sorted(set(LIB_UNITS) | set(PROBE_UNITS)):
        units.append((CSRC / f"{unit}.hip", OBJ_DIR / f"{unit}.o", []))
    jobs = jobs or min(len(units) + 1, max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [cc, *flags, *defs, "-c", str(src), "-o", str(obj)], verbose)
                for src, obj, defs in units]
        futs.append(ex.submit(_run, pyext_command(), verbose))
        for f in futs:
            f.result()
    os.replace(pyext_path().with_suffix(".so.tmp"), pyext_path())
    _link(cc, units, LIB_PATH, probe=False, verbose=verbose)
    _link(cc, units, PROBE_LIB_PATH, probe=True, verbose=verbose)
    return LIB_PATH


def _link(cc: str, units, lib: Path, *, probe: bool, verbose: bool, extra=()) -> None:
    """Links libfagq.so (every unit but the probes) or libfagq_probe.so (the
    probes and the device check) from the compiled units."""
    if probe:
        objs = [str(o) for src, o, _ in units if src.stem in PROBE_UNITS]
    else:
        objs = [str(o) for src, o, _ in units if src.stem != "fagq_probe"]
    tmp = lib.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *extra, "-o", str(tmp), *objs],
         verbose)
    os.replace(tmp, lib)


def sanitizer_runtime() -> Path:
    """The shared AddressSanitizer runtime of hipcc's clang (preloaded into a
    Python process that loads a sanitizer build)."""
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    found = sorted((rocm / "llvm" / "lib" / "clang").glob("*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise RuntimeError("clang's AddressSanitizer runtime not found under ROCm")
    return found[-1]


def build_variant(name: str, *, defines: tuple[str, ...] = (), sanitize: bool = False,
                  verbose: bool = False) -> Path:
    """A test-only build of the same sources into _build/<name>/libfagq.so (and
    libfagq_probe.so beside it), with
    extra -D defines (e.g. FAGQ_TEST_LAUNCH_FAILURE) and, with `sanitize`,
    AddressSanitizer and UndefinedBehaviorSanitizer on every host function
    (the argument validation, route table and host-side diagnostics; the
    device code is compiled as usual).  Never the library the package loads."""
    out_dir = OBJ_DIR / name
    out_dir.mkdir(parents=True, exist_ok=True)
    cc = hipcc()
    flags = [*device_flags(), *[f"-D{d}" for d in defines]]
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host",
           "-fno-omit-frame-pointer", "-Xarch_host", "-g"] if sanitize else []
    units: list[tuple[Path, Path, list[str]]] = []
    for q, sf in INST_COMBOS:
        units.append((CSRC / "fagq_inst.hip", out_dir / f"fagq_inst_q{q}_s{sf}.o",
                      [f"-DFAGQ_QF={q}", f"-DFAGQ_SF={sf}"]))
        units.append((CSRC / "fagq_inst_typed.hip", out_dir / f"fagq_inst_typed_q{q}_s{sf}.o",
                      [f"-DFAGQ_QF={q}", f"-DFAGQ_SF={sf}"]))
    for unit in sorted(set(LIB_UNITS) | set(PROBE_UNITS)):
        units.append((CSRC / f"{unit}.hip", out_dir / f"{unit}.o", []))
    with ThreadPoolExecutor(max_workers=min(len(units), max(1, min(16, os.cpu_count() or 1)))) as ex:
        futs = [ex.submit(_run, [cc, *flags, *san, *defs, "-c", str(src), "-o", str(obj)], verbose)
                for src, obj, defs in units]
        for f in futs:
            f.result()
    lib = out_dir / "libfagq.so"
    link_san = ["-fsanitize=address", "-fsanitize=undefined", "-shared-libsan"] if sanitize else []
    _link(cc, units, lib, probe=False, verbose=verbose, extra=link_san)
    _link(cc, units, out_dir / "libfagq_probe.so", probe=True, verbose=verbose, extra=link_san)
    return lib


if __name__ == "__main__":
    print(build(verbose=True))
