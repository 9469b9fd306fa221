"""The drop-in boundary from a plain C host: tests/c_abi/fagq_c_check (built
by `python __graft_entry__.py build`) calls fagq_launch through
include/fagq.h with no Python or torch in its process, and its outputs must
equal the CPU oracle's bit for bit; it also checks that argument errors come
back as status codes."""
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.compare import compare
from tests.gpu_util import note, run_ref

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "c_abi" / "fagq_c_check"


def test_c_host_calls_the_operator(pkg, gpu, tmp_path):
    if not EXE.exists():
        pytest.skip("tests/c_abi/fagq_c_check is not built (python __graft_entry__.py build)")
    M, D = 96, 7168
    g = torch.Generator().manual_seed(21)
    x = torch.randn(M, D, generator=g).bfloat16()
    r = torch.randn(M, D, generator=g).bfloat16()
    w = (1.0 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    for name, t in (("x.bin", x), ("residual.bin", r), ("gamma.bin", w)):
        (tmp_path / name).write_bytes(t.view(torch.uint16).numpy().tobytes())
    note(f"c host: M={M} D={D} fp8 f32 col-major, norm_out")
    p = subprocess.run([str(EXE), str(M), str(D), str(tmp_path)], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 0, p.stderr + p.stdout
    assert "ok" in p.stdout
    got = {"residual_out": np.fromfile(tmp_path / "residual_out.bin", dtype=np.uint16).reshape(M, D),
           "norm_out": np.fromfile(tmp_path / "norm_out.bin", dtype=np.uint16).reshape(M, D),
           "q": np.fromfile(tmp_path / "q.bin", dtype=np.uint8).reshape(M, D),
           "scale": np.fromfile(tmp_path / "scale.bin", dtype=np.float32).reshape(D // 128, M)}
    want = run_ref(x, r, w, 128, "fp8", False, True, with_norm=True)
    st = compare(got, want, fp8=True, ue8m0=False, label="c host")
    assert st["exact"], st
