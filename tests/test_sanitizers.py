"""The CPU tests of the host code under AddressSanitizer and
UndefinedBehaviorSanitizer.

The library is rebuilt with both sanitizers on every host function (argument
validation, route table, host-side diagnostics; device code as usual) and
the C oracle with clang's; a child pytest then runs the CPU tests of the
C ABI, the scale addressing, the oracle and the multi-input form against
those builds, with clang's shared ASan runtime preloaded.  Any sanitizer
report ends the child with an error, which fails this test."""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]

CHILD_TESTS = ["tests/test_boundary.py", "tests/test_scale_offsets.py", "tests/test_oracle.py",
               "tests/test_parts.py", "tests/test_golden.py", "tests/test_gemm_oracle.py",
               "tests/test_dsa_oracle.py", "tests/test_mla_oracle.py"]


@pytest.mark.skipif(os.environ.get("FAGQ_TEST_LIBRARY") is not None,
                    reason="already inside the sanitizer run")
def test_cpu_tests_pass_under_asan_and_ubsan(pkg):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a host-code check: CPU-only hosts run it")
    if not (shutil.which("hipcc") or Path("/opt/rocm/bin/hipcc").exists()):
        pytest.skip("hipcc not available")
    import __graft_entry__ as ge
    from oracle import build as oracle_build
    build = ge._load_module("fagq_mi355x_build", ge.PKG_DIR / "build.py")
    lib = build.build_variant("sanitize", sanitize=True)
    orc = oracle_build.build_sanitized()
    runtime = build.sanitizer_runtime()
    # Both builds are instrumented (they call the sanitizers' report hooks).
    for so in (lib, lib.parent / "libfagq_probe.so", orc):
        syms = subprocess.run(["nm", "-D", str(so)], capture_output=True, text=True).stdout
        assert "__asan_report" in syms and "__ubsan_handle" in syms, so
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": str(runtime),
        # Python and torch are not instrumented: leaks and ODR checks of
        # uninstrumented code are not findings about this code.
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:detect_odr_violation=0:"
                        "alloc_dealloc_mismatch=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "FAGQ_TEST_LIBRARY": str(lib),
        "FAGQ_TEST_PROBE_LIBRARY": str(lib.parent / "libfagq_probe.so"),
        "FAGQ_TEST_ORACLE_LIBRARY": str(orc),
    })
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        "-m", "not gpu", *CHILD_TESTS], cwd=REPO, env=env, capture_output=True,
                       text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert "passed" in r.stdout and "AddressSanitizer" not in tail and "runtime error" not in tail
