"""GPU parity of the HIP library against the CPU oracle, through the C ABI.

Bar: residual_out and norm_out bit-exact, fp32 scales within 1e-6
relative, codes equal except one-step differences on <= 0.01 % of elements
(oracle.compare).  Because the library and the oracle evaluate the same
exactly-rounded definition, the tests also record whether every output was
bit-identical."""
import math

import numpy as np
import pytest
import torch

from oracle.compare import compare
from tests.gpu_util import FMTS, note, run_gpu, run_ref

pytestmark = pytest.mark.gpu


def inputs(M, D, seed=0, scale=1.0, dist="normal"):
    g = torch.Generator().manual_seed(seed)
    if dist == "student_t":
        def draw(shape):
            z = torch.randn(shape, generator=g)
            chi2 = sum(torch.randn(shape, generator=g) ** 2 for _ in range(3))
            return 0.5 * z / torch.sqrt(chi2 / 3.0)
    else:
        def draw(shape):
            return torch.randn(shape, generator=g)
    x = (scale * draw((M, D))).bfloat16()
    r = (scale * draw((M, D))).bfloat16()
    w = (1.0 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    return x, r, w


def check(pkg, dev, x, r, w, G=128, fmt="fp8", ue8m0=False, col=False, with_norm=False,
          label="", **kw):
    note(f"case {label}: M={x.shape[0]} D={x.shape[1]} G={G} {fmt} ue8m0={ue8m0} "
         f"col={col} norm={with_norm} {kw}")
    gpu = run_gpu(pkg, dev, x, r, w, G, fmt, ue8m0, col, with_norm=with_norm, **kw)
    ref = run_ref(x, r, w, G, fmt, ue8m0, col, with_norm=with_norm)
    return compare(gpu, ref, fp8=fmt == "fp8", ue8m0=ue8m0, label=label), gpu


@pytest.mark.parametrize("name", ["cpu_ref_128x4096", "prefill_4096x4096", "dsv3_16384x7168",
                                  "decode_1x8192", "decode_4x8192", "decode_16x8192",
                                  "decode_32x8192", "ue8m0_8192x5120"])
def test_baseline_configs_full_size(pkg, gpu, name):
    from fagq_mi355x.workloads import CONFIGS, make_inputs
    w = CONFIGS[name]
    x, r, g = make_inputs(w)
    fmt = "fp8" if w.out_dtype == torch.float8_e4m3fn else f"int8_{w.rounding}"
    st, _ = check(pkg, gpu, x, r, g, w.group_size, fmt, w.scale_ue8m0, w.scale_col_major,
                  label=name)
    note(f"  {name}: {st}")
    assert st["exact"], st


@pytest.mark.parametrize("name", ["ref4_16384x7168", "ref4_4096x4096"])
def test_reference_mode_full_size(pkg, gpu, name):
    """The reference's own output mode at full size: norm_out written, int8
    codes by truncation, fp32 row-major scales (the bench's ref4 workloads)."""
    from fagq_mi355x.workloads import REFERENCE_MODE_CONFIGS, make_inputs
    w = REFERENCE_MODE_CONFIGS[name]
    x, r, g = make_inputs(w)
    st, _ = check(pkg, gpu, x, r, g, w.group_size, f"int8_{w.rounding}", w.scale_ue8m0,
                  w.scale_col_major, with_norm=w.norm, label=name)
    note(f"  {name}: {st}")
    assert st["exact"], st


@pytest.mark.parametrize("G", [64, 128, 256])
@pytest.mark.parametrize("fmt", ["fp8", "int8_rne", "int8_trunc"])
@pytest.mark.parametrize("ue8m0", [False, True])
@pytest.mark.parametrize("col", [False, True])
def test_format_matrix(pkg, gpu, G, fmt, ue8m0, col):
    x, r, w = inputs(37, 3072, seed=G, scale=2.0)
    st, _ = check(pkg, gpu, x, r, w, G, fmt, ue8m0, col, with_norm=(G == 128),
                  label="format-matrix")
    assert st["exact"], st


@pytest.mark.parametrize("D,G", [(7168, 128), (5120, 256), (4160, 64), (8192, 128), (1536, 64)])
def test_every_launch_mapping(pkg, gpu, D, G):
    """Every legal (waves_per_row, rows_per_block, row_group_mode, xcd_remap)
    gives identical outputs, including row counts that leave the last
    workgroup's row groups partly empty (M = 19)."""
    M = 19
    x, r, w = inputs(M, D, seed=D)
    ref = None
    steps = math.ceil(D / 512)
    n = 0
    for wpr in range(1, 17):
        ns = math.ceil(steps / wpr)
        if ns > 4:
            continue
        for rpb in (1, 2, 3, 4, 8, 16):
            if wpr * rpb > 16:
                continue
            for mode in (0, 1, 2):
                if mode and wpr * ns > 16:
                    continue
                if mode == 2 and rpb not in (2, 4):
                    continue
                for remap in ((0, 1, 2, 8) if mode == 0 else (0, 4)):
                    st, gpu_out = check(pkg, gpu, x, r, w, G, "fp8", col=True,
                                        mapping=(wpr, rpb, mode, remap),
                                        label=f"map wpr={wpr} rpb={rpb} mode={mode} remap={remap}")
                    assert st["exact"], st
                    if ref is None:
                        ref = gpu_out
                    for k in ref:
                        assert np.array_equal(ref[k], gpu_out[k]), (wpr, rpb, mode, remap, k)
                    n += 1
    assert n >= 20


@pytest.mark.parametrize("mode,rpb", [(1, 2), (1, 3), (2, 2), (2, 4)])
@pytest.mark.parametrize("M", [37, 8])
def test_shared_modes_all_formats(pkg, gpu, mode, rpb, M):
    """Gamma shared through LDS (mode 1) and wide column-major scale stores (mode 2)
    in every code and scale format, with norm_out, for M a multiple of the rows
    per workgroup (8) and not (37: the last workgroup stores row by row)."""
    x, r, w = inputs(M, 5120, seed=mode * 10 + rpb, scale=3.0)
    for fmt in ("fp8", "int8_rne", "int8_trunc"):
        for ue in (False, True):
            for wpr in (3, 5):
                if wpr * rpb > 16:
                    continue
                st, _ = check(pkg, gpu, x, r, w, 128, fmt, ue8m0=ue, col=(mode == 2 or ue),
                              with_norm=True, mapping=(wpr, rpb, mode, 0),
                              label=f"mode={mode} rpb={rpb} wpr={wpr}")
                assert st["exact"], st


@pytest.mark.parametrize("ue8m0", [False, True])
@pytest.mark.parametrize("offset", [1, 2, 3])
def test_wide_scales_misaligned_pointer(pkg, gpu, ue8m0, offset):
    """Mode 2 with a scale pointer not aligned to the wide store: every row stores
    its own scales, and the outputs are unchanged."""
    x, r, w = inputs(64, 7168, seed=offset)
    st, gpu_out = check(pkg, gpu, x, r, w, 128, "fp8", ue8m0=ue8m0, col=True,
                        mapping=(4, 2, 2, 8), scale_offset=offset, label=f"wide offset={offset}")
    assert st["exact"], st


def test_occupancy_cap_gives_the_same_bits(pkg, gpu):
    """Reserving dynamic LDS per workgroup (fewer workgroups per CU) changes nothing."""
    x, r, w = inputs(300, 7168, seed=3)
    outs = []
    for lds in (0, 49152, 65536):
        st, gpu_out = check(pkg, gpu, x, r, w, 128, "fp8", col=True, mapping=(7, 1, 0, 8, lds),
                            label=f"lds={lds}")
        assert st["exact"], st
        outs.append(gpu_out)
    for o in outs[1:]:
        for k in o:
            assert np.array_equal(o[k], outs[0][k])


@pytest.mark.parametrize("M,D,G", [(1, 192, 64), (5, 640, 128), (130, 4160, 64), (3, 8448, 128),
                                   (7, 12288, 256), (2, 16384, 128), (3, 32768, 128),
                                   (1000, 1536, 128), (257, 7168, 128), (33, 128, 128)])
def test_ragged_and_large_rows(pkg, gpu, M, D, G):
    x, r, w = inputs(M, D, seed=M + D)
    for fmt in ("fp8", "int8_rne"):
        st, _ = check(pkg, gpu, x, r, w, G, fmt, col=(M % 2 == 1), label="ragged")
        assert st["exact"], st


def test_zero_rows_is_a_no_op(pkg, gpu):
    x = torch.empty(0, 4096, dtype=torch.bfloat16, device=gpu)
    q = torch.empty(0, 4096, dtype=torch.float8_e4m3fn, device=gpu)
    sc = torch.empty(0, 32, device=gpu)
    out = pkg.fused_add_rmsnorm_group_quant(x, x, torch.ones(4096, dtype=torch.bfloat16, device=gpu),
                                            torch.empty_like(x), None, q, sc, 1e-6, 128)
    assert out[2] is q and out[3] is sc


def test_in_place_residual_update(pkg, gpu):
    x, r, w = inputs(64, 7168, seed=3)
    st, _ = check(pkg, gpu, x, r, w, 128, "fp8", inplace=True, label="inplace")
    assert st["exact"], st


def test_reference_signature_four_outputs(pkg, gpu):
    """int8 x_q with the reference's signature: truncating codes and norm_out."""
    x, r, w = inputs(96, 4096, seed=4)
    st, _ = check(pkg, gpu, x, r, w, 128, "int8_trunc", with_norm=True, label="ref-4-output")
    assert st["exact"], st
    st, _ = check(pkg, gpu, x, r, w, 256, "int8_trunc", with_norm=True, label="ref-4-output-g256")
    assert st["exact"], st


def test_special_rows(pkg, gpu):
    M, D = 12, 4096
    x, r, w = inputs(M, D, seed=5)
    x[0] = 0
    r[0] = 0                                    # all-zero row
    x[1] = 0
    r[1] = 0
    x[1, 777] = 3.0                             # one-hot row
    x[2] = 1.5
    r[2] = 0                                    # constant row
    x[3] = 1.0e38
    r[3] = 0                                    # near the bf16 maximum
    x[4] = 1e-39                                # bf16 and fp32 subnormals
    r[4] = 2e-39
    x[5, ::2] = 0                               # half-zero row
    x[6, :128] = 0
    r[6, :128] = 0                              # an all-zero group in a normal row
    x[7] *= 1e4                                 # large dynamic range
    x[8, 5] = 60000.0                           # one outlier in a group
    for fmt in ("fp8", "int8_rne", "int8_trunc"):
        for ue in (False, True):
            st, _ = check(pkg, gpu, x, r, w, 128, fmt, ue8m0=ue, with_norm=True, label="special")
            assert st["exact"], st


def test_heavy_tailed_inputs(pkg, gpu):
    x, r, w = inputs(256, 5120, seed=6, dist="student_t")
    st, _ = check(pkg, gpu, x, r, w, 128, "fp8", ue8m0=True, col=True, label="student-t")
    assert st["exact"], st


def test_side_stream(pkg, gpu):
    x, r, w = inputs(128, 7168, seed=7)
    s = torch.cuda.Stream(device=gpu)
    st, _ = check(pkg, gpu, x, r, w, 128, "fp8", col=True, stream=s, label="side-stream")
    assert st["exact"], st


def test_functional_form(pkg, gpu):
    x, r, w = inputs(40, 4096, seed=8)
    note("case functional form")
    xd, rd, wd = x.to(gpu), r.to(gpu), w.to(gpu)
    ro, q, sc = pkg.fused_add_rmsnorm_group_quant_fn(xd, rd, wd, 1e-6, 128, torch.int8,
                                                     scale_col_major=True)
    torch.cuda.synchronize(gpu)
    assert sc.shape == (40, 32) and sc.stride() == (1, 40)
    ref = run_ref(x, r, w, 128, "int8_rne", col=True)
    gpu_out = {"residual_out": ro.cpu().view(torch.uint16).numpy(),
               "q": q.cpu().view(torch.uint8).numpy(),
               "scale": np.ascontiguousarray(sc.t().cpu().numpy())}
    st = compare(gpu_out, ref, fp8=False, ue8m0=False)
    assert st["exact"], st
    ro2, _, _ = pkg.fused_add_rmsnorm_group_quant_fn(xd, rd, wd, inplace_residual=True)
    assert ro2 is rd


def test_python_layer_rejects_bad_gpu_arguments(pkg, gpu):
    M, D = 8, 1024
    x = torch.zeros(M, D, dtype=torch.bfloat16, device=gpu)
    g = torch.ones(D, dtype=torch.bfloat16, device=gpu)
    q = torch.empty(M, D, dtype=torch.float8_e4m3fn, device=gpu)
    sc = torch.empty(M, D // 128, device=gpu)
    f = pkg.fused_add_rmsnorm_group_quant
    with pytest.raises(TypeError):
        f(x.float(), x, g, x, None, q, sc, 1e-6, 128)
    with pytest.raises(ValueError):
        f(x, x, g, x.t().contiguous().t(), None, q, sc, 1e-6, 128)   # non-contiguous output
    with pytest.raises(ValueError):
        f(x, x, g[:512], torch.empty_like(x), None, q, sc, 1e-6, 128)
    with pytest.raises(ValueError):
        f(x, x, g, torch.empty_like(x), None, q, sc, 1e-6, 100)
    with pytest.raises(ValueError):
        f(x, x, g, torch.empty_like(x), None, q, torch.empty(M, 4, device=gpu), 1e-6, 128)
    from fagq_mi355x import _lib
    with pytest.raises(_lib.FagqError) as e:
        f(x, x, g, torch.empty_like(x), None, q, torch.empty(M, 2, device=gpu), 1e-6, 512)
    assert e.value.status == 3
    with pytest.raises(_lib.FagqError) as e:
        f(x, x, g, torch.empty_like(x), None, q, sc, -1.0, 128)
    assert e.value.status == 6


@pytest.mark.parametrize("M,D,fmt,ue8m0,col,with_norm", [
    (1, 8192, "int8_rne", False, False, False), (33, 4096, "int8_trunc", True, True, True),
    (512, 7168, "fp8", False, True, False), (300, 5120, "fp8", True, False, True)])
def test_cpython_binding_matches_ctypes_path(pkg, gpu, M, D, fmt, ue8m0, col, with_norm):
    """The operator's per-call CPython binding and the ctypes path launch the same
    kernel: bit-identical outputs, and the binding is the one the operator uses."""
    from fagq_mi355x import _lib, ops
    assert _lib.fast_launch() is not None
    note(f"binding vs ctypes M={M} D={D} {fmt} ue8m0={ue8m0} col={col} norm={with_norm}")
    x, r, w = inputs(M, D, seed=M + D)
    qdt, rounding = FMTS[fmt][0], FMTS[fmt][1]
    xd, rd, wd = x.to(gpu), r.to(gpu), w.to(gpu)
    outs = []
    for use_fast in (True, False):
        ro = torch.empty_like(rd)
        no = torch.empty_like(rd) if with_norm else None
        q = torch.empty(M, D, dtype=qdt, device=gpu)
        sc = pkg.empty_scales(M, D // 128, ue8m0=ue8m0, col_major=col, device=gpu)
        saved = (_lib._fast, _lib._fast_tried)
        if not use_fast:
            _lib._fast, _lib._fast_tried = None, True
        try:
            ops.fused_add_rmsnorm_group_quant(xd, rd, wd, ro, no, q, sc, 1e-6, 128,
                                              rounding=rounding if qdt == torch.int8 else None)
        finally:
            _lib._fast, _lib._fast_tried = saved
        torch.cuda.synchronize(gpu)
        outs.append([t.cpu().view(torch.uint8) for t in (ro, q, sc.contiguous()) + ((no,) if with_norm else ())])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
