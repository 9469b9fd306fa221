"""GPU parity of the multi-input form (fagq_launch_parts) against the CPU
oracle (oracle.fagq_parts), through the C ABI.  Same bar as the
single-input tests (oracle.compare); the outputs are also expected to be
bit-identical, and with one part identical to the single-input kernel's."""
import numpy as np
import pytest
import torch

import oracle
from oracle.compare import compare
from tests.gpu_util import note

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def inputs(nparts, M, D, seed=0):
    g = torch.Generator().manual_seed(seed)
    parts = [torch.randn(M, D, generator=g).bfloat16() for _ in range(nparts)]
    r = torch.randn(M, D, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    return parts, r, w


def run(pkg, dev, parts, r, w, G=128, out_dtype=FP8, col=True, ue8m0=False, rounding="rne",
        inplace=False):
    pd = [p.to(dev) for p in parts]
    rd, wd = r.to(dev), w.to(dev)
    ro, q, sc = pkg.fused_reduce_add_rmsnorm_group_quant(
        pd, rd, wd, 1e-6, G, out_dtype, scale_col_major=col, scale_ue8m0=ue8m0,
        rounding=rounding, inplace_residual=inplace)
    torch.cuda.synchronize()
    return {"residual_out": ro.cpu().view(torch.uint16).numpy(),
            "q": q.cpu().view(torch.uint8).numpy(),
            "scale": np.ascontiguousarray((sc.t() if col else sc).cpu().numpy())}


def ref(parts, r, w, G=128, out_dtype=FP8, col=True, ue8m0=False, rounding="rne"):
    u16 = lambda t: t.contiguous().view(torch.uint16).numpy()
    qf = oracle.Q_FP8 if out_dtype == FP8 else oracle.Q_INT8
    return oracle.fagq_parts([u16(p) for p in parts], u16(r), u16(w), 1e-6, G, qf,
                             oracle.S_UE8M0 if ue8m0 else oracle.S_F32,
                             oracle.L_COL if col else oracle.L_ROW,
                             oracle.R_RNE if rounding == "rne" else oracle.R_TRUNC)


CASES = [  # nparts, M, D, G, out dtype, col, ue8m0, rounding
    (1, 300, 7168, 128, FP8, True, False, "rne"),
    (2, 300, 7168, 128, FP8, True, False, "rne"),
    (3, 129, 4096, 128, FP8, False, False, "rne"),
    (4, 257, 7168, 128, FP8, True, True, "rne"),
    (8, 300, 7168, 128, FP8, True, False, "rne"),
    (8, 64, 16384, 128, FP8, True, False, "rne"),      # 2 steps per wave
    (5, 33, 640, 64, torch.int8, False, False, "trunc"),  # ragged row, small D (rows share a workgroup)
    (2, 17, 8192, 256, torch.int8, False, True, "rne"),
    (7, 1, 5120, 128, FP8, True, True, "rne"),
    # 6-8 partials and 12-16 steps: 4-step waves
    (6, 64, 6144, 128, FP8, False, True, "rne"),           # 3 waves of 4 steps
    (6, 100, 6400, 128, torch.int8, False, False, "rne"),  # last wave 1.5 steps
    (7, 33, 6656, 64, torch.int8, True, False, "trunc"),
    (8, 50, 8192, 256, FP8, True, True, "rne"),
]


@pytest.mark.parametrize("nparts,M,D,G,dt,col,ue,rnd", CASES)
def test_parts_parity(pkg, gpu, nparts, M, D, G, dt, col, ue, rnd):
    note(f"parts P={nparts} M={M} D={D} G={G} {dt} col={col} ue8m0={ue} {rnd}")
    parts, r, w = inputs(nparts, M, D, seed=nparts * 100 + M)
    got = run(pkg, gpu, parts, r, w, G, dt, col, ue, rnd)
    want = ref(parts, r, w, G, dt, col, ue, rnd)
    st = compare(got, want, fp8=dt == FP8, ue8m0=ue, label=f"parts P={nparts}")
    assert st["exact"], st


def test_one_part_matches_single_input_kernel(pkg, gpu):
    parts, r, w = inputs(1, 200, 7168, seed=9)
    note("parts P=1 vs single-input kernel")
    got = run(pkg, gpu, parts, r, w)
    ro, q, sc = pkg.fused_add_rmsnorm_group_quant_fn(parts[0].to(gpu), r.to(gpu), w.to(gpu),
                                                     1e-6, 128, FP8, scale_col_major=True)
    torch.cuda.synchronize()
    assert np.array_equal(got["residual_out"], ro.cpu().view(torch.uint16).numpy())
    assert np.array_equal(got["q"], q.cpu().view(torch.uint8).numpy())
    assert np.array_equal(got["scale"], sc.t().contiguous().cpu().numpy())


def test_parts_in_place_residual(pkg, gpu):
    parts, r, w = inputs(4, 96, 7168, seed=3)
    note("parts in place")
    got = run(pkg, gpu, parts, r, w, inplace=True)
    want = ref(parts, r, w)
    assert compare(got, want, fp8=True, ue8m0=False)["exact"]


@pytest.mark.parametrize("name", ["tp8_shard_2048x7168", "tp4_shard_4096x7168"])
def test_parts_tp_shards_full_size(pkg, gpu, name):
    """The headline shape sharded over 8 or 4 ranks: 2048 rows x 7168 with 8
    partial sums (4-step waves), 4096 rows with 4 (2-step waves)."""
    from fagq_mi355x.workloads import PARTS_CONFIGS, make_parts_inputs
    w = PARTS_CONFIGS[name]
    note(f"parts full size {w.name}")
    parts, r, g = make_parts_inputs(w)
    got = run(pkg, gpu, parts, r, g)
    want = ref(parts, r, g)
    assert compare(got, want, fp8=True, ue8m0=False)["exact"]


def test_parts_zero_rows_and_errors(pkg, gpu):
    parts, r, w = inputs(2, 0, 1024)
    ro, q, sc = pkg.fused_reduce_add_rmsnorm_group_quant([p.to(gpu) for p in parts], r.to(gpu),
                                                         w.to(gpu), 1e-6, 128)
    assert ro.shape == (0, 1024) and q.shape == (0, 1024)
    with pytest.raises(ValueError):
        pkg.fused_reduce_add_rmsnorm_group_quant([], r.to(gpu), w.to(gpu))
    with pytest.raises(ValueError):
        pkg.fused_reduce_add_rmsnorm_group_quant([parts[0].to(gpu)] * 9, r.to(gpu), w.to(gpu))
    p2, r2, w2 = inputs(2, 4, 32768)
    with pytest.raises(pkg.FagqError):
        pkg.fused_reduce_add_rmsnorm_group_quant([p.to(gpu) for p in p2], r2.to(gpu), w2.to(gpu))
