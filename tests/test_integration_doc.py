"""The ctypes stubs INTEGRATION.md shows a maintainer of the reference: every
Python block that declares `_fagq.<function>.argtypes` runs here against the
built libfagq.so (CPU only, no call reaches the device), and each declaration
must match the library's own binding (`_lib.SIGNATURES`, itself checked
against include/*.h by test_boundary.py)."""
import ctypes
import re
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def stub_blocks():
    text = (REPO / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    return [b for b in blocks if ".argtypes" in b]


def test_stubs_match_the_library(pkg, lib):
    from fagq_mi355x import _lib
    import torch
    blocks = stub_blocks()
    assert blocks, "INTEGRATION.md shows no ctypes stub"
    ns = {"ctypes": ctypes, "torch": torch}
    declared = set()
    for b in blocks:
        # The stub loads the library from a placeholder path; load the built one.
        code = re.sub(r'ctypes\.CDLL\("[^"]*"\)', "ctypes.CDLL(LIB_PATH)", b)
        ns["LIB_PATH"] = str(_lib.LIB_PATH)
        exec(compile(code, "INTEGRATION.md", "exec"), ns)
        declared |= set(re.findall(r"_fagq\.(\w+)\.argtypes\s*=", b))
    f = ns["_fagq"]
    assert "fagq_launch" in declared and "fagq_launch_typed" in declared
    for name in sorted(declared):
        fn = getattr(f, name)
        want_args, want_res = _lib.SIGNATURES[name]
        assert list(fn.argtypes) == list(want_args), name
        assert fn.restype == want_res, name
    # The reference-side function the main stub defines.
    assert callable(ns["fused_add_rmsnorm_group_quant"])
