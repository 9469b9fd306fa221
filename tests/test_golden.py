"""Golden fixtures (tests/golden/fagq_golden.npz, written by
tests/golden/make_golden.py from the pinned C oracle): the oracle must
reproduce them bit for bit on the CPU, and the GPU library through the C ABI
on the GPU."""
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "fagq_golden.npz"


def cases():
    data = np.load(GOLDEN)          # allow_pickle=False (default)
    names = sorted({k.split(".")[0] for k in data.files if "." in k})
    eps = float(data["eps"][0])
    out = []
    for n in names:
        M, D, G, qf, sf, lay, rnd, wn = (int(v) for v in data[f"{n}.meta"])
        exp = {k: data[f"{n}.{k}"] for k in ("residual_out", "q", "scale", "norm_out")
               if f"{n}.{k}" in data.files}
        out.append(dict(name=n, M=M, D=D, G=G, qf=qf, sf=sf, lay=lay, rnd=rnd, wn=bool(wn),
                        eps=eps, x=data[f"{n}.x"], r=data[f"{n}.residual"],
                        g=data[f"{n}.gamma"], exp=exp))
    return out


CASES = cases()


@pytest.mark.parametrize("c", CASES, ids=[c["name"] for c in CASES])
def test_oracle_reproduces_golden(c):
    got = oracle.fagq(c["x"], c["r"], c["g"], c["eps"], c["G"], c["qf"], c["sf"], c["lay"],
                      c["rnd"], c["wn"])
    for k, v in c["exp"].items():
        assert np.array_equal(got[k], v), (c["name"], k)


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=[c["name"] for c in CASES])
def test_gpu_reproduces_golden(pkg, gpu, c):
    import torch
    from tests.gpu_util import note, run_gpu
    fmt = "fp8" if c["qf"] == oracle.Q_FP8 else ("int8_rne" if c["rnd"] == oracle.R_RNE else "int8_trunc")
    note(f"case golden {c['name']}")
    as_bf16 = lambda a: torch.from_numpy(a.astype(np.int16)).view(torch.bfloat16)
    got = run_gpu(pkg, gpu, as_bf16(c["x"]), as_bf16(c["r"]), as_bf16(c["g"]), c["G"], fmt,
                  ue8m0=c["sf"] == oracle.S_UE8M0, col=c["lay"] == oracle.L_COL, eps=c["eps"],
                  with_norm=c["wn"])
    for k, v in c["exp"].items():
        assert np.array_equal(got[k], v), (c["name"], k, int(np.count_nonzero(got[k] != v)))
