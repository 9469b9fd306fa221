"""The C ABI boundary and the Python host layer, without a GPU: the libraries
load and export everything include/*.h declares (libfagq_probe.so the
measurement probes of fagq_probe.h, libfagq.so the rest), the route table
keeps its invariants, and every argument error is reported before any device
work."""
import ctypes
import math
import re
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
HEADERS = sorted((REPO / "include").glob("*.h"))


PROBE_HEADER = "fagq_probe.h"


def declared_functions(probe=None):
    """FAGQ_API functions of every header; probe=True: fagq_probe.h only,
    probe=False: every other header."""
    names = []
    for h in HEADERS:
        if probe is not None and (h.name == PROBE_HEADER) != probe:
            continue
        text = h.read_text()
        names += re.findall(r"FAGQ_API\s+[\w\s\*]+?\b(\w+)\s*\(", text)
    return names


def test_headers_declare_the_abi():
    names = declared_functions()
    assert "fagq_launch" in names and "fagq_query_route" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol(pkg, lib, probe_lib):
    from fagq_mi355x import _lib
    for name in declared_functions(probe=False):
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
    assert set(_lib.SIGNATURES) == set(declared_functions(probe=False))
    for name in declared_functions(probe=True):
        assert hasattr(probe_lib, name), name
        assert name in _lib.PROBE_SIGNATURES, name
    assert set(_lib.PROBE_SIGNATURES) == set(declared_functions(probe=True))


def test_probes_are_not_in_the_drop_in_library(lib):
    # The measurement probes live in libfagq_probe.so only.
    for name in declared_functions(probe=True):
        assert not hasattr(lib, name), name


def test_version_and_status_strings(lib):
    assert lib.fagq_version() == 10000
    for st in range(0, 10):
        s = lib.fagq_status_string(st).decode()
        assert s and s != "unknown status"
    assert lib.fagq_status_string(-1).decode() == "HIP runtime error"


SHAPES = [(M, D) for M in (1, 4, 16, 32, 100, 128, 512, 4096, 16384) for D in
          (128, 640, 4096, 5120, 7168, 8192, 8448, 16384, 32768)]


@pytest.mark.parametrize("M,D", SHAPES)
@pytest.mark.parametrize("ue8m0,col", [(False, False), (False, True), (True, True)])
def test_route_invariants(pkg, M, D, ue8m0, col):
    r = pkg.route_for(M, D, 128, scale_ue8m0=ue8m0, scale_col_major=col)
    wpr, ns, rpb, mode = (r["waves_per_row"], r["steps_per_wave"], r["rows_per_block"],
                          r["row_group_mode"])
    steps = math.ceil(D / 512)
    assert 1 <= wpr <= 16 and 1 <= ns <= 4 and rpb >= 1 and mode in (0, 1, 2)
    assert wpr * ns >= steps > (wpr - 1) * ns          # every wave owns >= 1 column
    assert r["block_threads"] == 64 * wpr * rpb <= 1024
    assert r["grid_blocks"] * rpb >= M > (r["grid_blocks"] - 1) * rpb
    assert r["lds_bytes"] in (0, 36864, 49152)
    if mode:
        assert wpr * ns <= 16                            # gamma fits the LDS buffer
    if mode == 2:
        assert col and rpb in (2, 4)
    prefill = M >= 1024
    if prefill and 12 <= steps <= 16:
        if col:
            # 5632 < D <= 8192, column-major: two rows per workgroup of 4-step
            # waves, shared gamma, wide scale stores, 16 rows per XCD chunk
            # (fp32) or 32 (ue8m0).
            assert (ns, rpb, mode, r["xcd_remap"]) == (4, 2, 2, 8 if not ue8m0 else 16)
        elif steps >= 15:
            assert (ns, rpb, mode) == (4, 2, 1)
        else:
            assert (ns, rpb, mode, r["lds_bytes"]) == (2, 1, 0, 49152)
    elif prefill and 5 <= steps <= 8:
        assert (wpr, ns, mode) == (steps, 1, 0)          # 1-step waves
    elif prefill and 2 <= steps <= 16:
        assert (ns, mode) == (2, 0)                      # prefill: 2-step waves
    if prefill and 9 <= steps <= 11:
        assert (ns, rpb, r["lds_bytes"]) == (2, 1, 36864)   # at most 4 workgroups per CU
    elif not (prefill and 12 <= steps <= 14 and not col):
        assert r["lds_bytes"] == 0
    if M <= 32 and D <= 8192:
        assert (wpr, ns, mode) == (steps, 1, 0)          # decode: one step per wave
    if not col:
        assert r["xcd_remap"] == 0


@pytest.mark.parametrize("args,status", [
    ((4, 4096, 100, 0, 0), 3), ((4, 4000, 128, 0, 0), 2), ((-1, 4096, 128, 0, 0), 2),
    ((4, 0, 128, 0, 0), 2), ((4, 65536, 128, 0, 0), 7), ((4, 4096, 128, 2, 0), 5),
    ((4, 4096, 128, 0, 2), 5),
])
def test_route_rejects_bad_shapes(lib, args, status):
    from fagq_mi355x import _lib
    r = _lib.Route()
    assert lib.fagq_query_route(*args, ctypes.byref(r)) == status
    # The typed query validates the shape the same way, before the dtypes.
    assert lib.fagq_query_route_typed(*args, 2, 2, ctypes.byref(r)) == status


TYPED_PAIRS = [(torch.float16, torch.float16), (torch.bfloat16, torch.float32),
               (torch.float16, torch.float32), (torch.float32, torch.float32)]


@pytest.mark.parametrize("M,D", [(1, 4096), (32, 8192), (4096, 4096), (8192, 5120),
                                 (16384, 7168), (16384, 16384)])
@pytest.mark.parametrize("at,rt", TYPED_PAIRS)
@pytest.mark.parametrize("ue8m0,col", [(False, False), (False, True), (True, True)])
def test_typed_routes(pkg, M, D, at, rt, ue8m0, col):
    """fp16 tensors take the bf16 operator's route; the pairs with an fp32
    tensor take the typed kernel's default mapping: independent rows, one row
    per workgroup when a row has 4 or more waves, and 1-step waves for
    prefill rows of 5-8 steps, 2-step waves otherwise (1 for decode)."""
    r = pkg.route_for(M, D, 128, scale_ue8m0=ue8m0, scale_col_major=col, x_dtype=at,
                      residual_dtype=rt)
    bf16 = pkg.route_for(M, D, 128, scale_ue8m0=ue8m0, scale_col_major=col)
    if at is torch.float16 and rt is torch.float16:
        assert r == bf16
        return
    steps = math.ceil(D / 512)
    prefill = M >= 1024
    ns = (1 if 5 <= steps <= 8 else 2) if prefill else 1
    ns = min(max(ns, math.ceil(steps / 16)), steps)
    wpr = math.ceil(steps / ns)
    rpb = 1 if wpr >= 4 else 4 // wpr
    assert (r["waves_per_row"], r["steps_per_wave"], r["rows_per_block"], r["row_group_mode"]) == \
        (wpr, ns, rpb, 0)
    assert r["block_threads"] == 64 * wpr * rpb
    assert r["grid_blocks"] == math.ceil(M / rpb)
    assert r["lds_bytes"] == (36864 if prefill and ns == 2 and rpb == 1 and 9 <= steps <= 11 else 0)


@pytest.mark.parametrize("M,D", [(1, 640), (33, 4096), (2048, 5632), (2048, 5760), (2048, 6144),
                                 (2048, 7168), (2048, 8192), (2048, 8320), (4096, 16384)])
@pytest.mark.parametrize("nparts", [1, 2, 4, 5, 6, 8])
def test_parts_routes(lib, M, D, nparts):
    """The multi-input form: 4-step waves for 6 or more partials at 12..16
    steps of 512 columns (5632 < D <= 8192), 2-step waves otherwise (1 step
    for rows of one step), independent rows, small rows sharing a workgroup."""
    from fagq_mi355x import _lib
    r = _lib.query_route_parts(M, D, 128, nparts, _lib.SCALE_F32, _lib.LAYOUT_COL_MAJOR)
    steps = math.ceil(D / 512)
    ns = 4 if nparts >= 6 and 12 <= steps <= 16 else min(2, steps)
    wpr = math.ceil(steps / ns)
    rpb = 1 if wpr >= 4 else 4 // wpr
    assert (r["waves_per_row"], r["steps_per_wave"], r["rows_per_block"], r["row_group_mode"]) == \
        (wpr, ns, rpb, 0)
    assert r["block_threads"] == 64 * wpr * rpb <= (512 if ns == 4 else 1024)
    assert r["grid_blocks"] == math.ceil(M / rpb)
    assert r["lds_bytes"] == 0


@pytest.mark.parametrize("args,status", [
    ((4, 4096, 128, 0, 0, 0), 2), ((4, 4096, 128, 9, 0, 0), 2), ((4, 16896, 128, 8, 0, 0), 7),
    ((4, 4096, 100, 8, 0, 0), 3), ((4, 4096, 128, 8, 2, 0), 5),
])
def test_parts_route_rejects_bad_arguments(lib, args, status):
    from fagq_mi355x import _lib
    r = _lib.Route()
    assert lib.fagq_query_route_parts(*args, ctypes.byref(r)) == status
    assert lib.fagq_query_route_parts(4096, 4096, 128, 8, 0, 0, None) == 1


def test_typed_route_rejects_unknown_pairs(lib):
    from fagq_mi355x import _lib
    r = _lib.Route()
    # (fp32 x, bf16 residual) and out-of-range codes are not element-type pairs.
    for at, rt in ((2, 0), (2, 1), (0, 1), (1, 0), (3, 3), (-1, 0)):
        assert lib.fagq_query_route_typed(4096, 4096, 128, 0, 0, at, rt, ctypes.byref(r)) == 5
    assert lib.fagq_query_route_typed(4096, 4096, 128, 0, 0, 0, 0, None) == 1
    with pytest.raises(TypeError):
        import fagq_mi355x
        fagq_mi355x.route_for(64, 4096, x_dtype=torch.int8)


# Fake, aligned, non-overlapping device addresses: validation never dereferences them.
BASE = 0x10_0000_0000


def fake(i):
    return ctypes.c_void_p(BASE + i * 0x1_0000_0000)


def call(lib, **kw):
    a = dict(x=fake(0), residual=fake(1), gamma=fake(2), residual_out=fake(3), norm_out=None,
             q=fake(4), scale=fake(5), M=8, D=4096, G=128, eps=1e-6, qf=1, sf=0, layout=0,
             rounding=0, stream=None)
    a.update(kw)
    return lib.fagq_launch(a["x"], a["residual"], a["gamma"], a["residual_out"], a["norm_out"],
                           a["q"], a["scale"], a["M"], a["D"], a["G"], a["eps"], a["qf"],
                           a["sf"], a["layout"], a["rounding"], a["stream"])


@pytest.mark.parametrize("kw,status", [
    (dict(x=None), 1), (dict(residual=None), 1), (dict(gamma=None), 1),
    (dict(residual_out=None), 1), (dict(q=None), 1), (dict(scale=None), 1),
    (dict(qf=2), 5), (dict(sf=2), 5), (dict(layout=2), 5), (dict(rounding=2), 5),
    (dict(qf=1, rounding=1), 5),                        # fp8 codes are RNE only
    (dict(G=32), 3), (dict(G=512), 3), (dict(D=4000), 2), (dict(M=-1), 2),
    (dict(D=65536), 7), (dict(eps=-1e-6), 6), (dict(eps=float("nan")), 6),
    (dict(eps=float("inf")), 6),
    (dict(x=ctypes.c_void_p(BASE + 8)), 4), (dict(gamma=ctypes.c_void_p(BASE + 0x2_0000_0004)), 4),
    (dict(q=ctypes.c_void_p(BASE + 0x4_0000_0004)), 4),
    (dict(scale=ctypes.c_void_p(BASE + 0x5_0000_0002)), 4),
    (dict(norm_out=ctypes.c_void_p(BASE + 0x6_0000_0008)), 4),
    (dict(q=ctypes.c_void_p(BASE + 0x1000)), 9),        # codes overlap x
    (dict(residual_out=ctypes.c_void_p(BASE + 0x1_0000_0000 + 0x100)), 9),   # partial overlap
    (dict(scale=fake(3)), 9),
    (dict(norm_out=fake(4)), 9),
    (dict(M=0), 0),                                     # no-op, device never touched
])
def test_launch_validation(lib, kw, status):
    assert call(lib, **kw) == status


def call_typed(lib, act, res, **kw):
    a = dict(x=fake(0), residual=fake(1), gamma=fake(2), residual_out=fake(3), norm_out=None,
             q=fake(4), scale=fake(5), M=8, D=4096, G=128, eps=1e-6, qf=1, sf=0, layout=0,
             rounding=0, stream=None)
    a.update(kw)
    return lib.fagq_launch_typed(a["x"], a["residual"], a["gamma"], a["residual_out"],
                                 a["norm_out"], a["q"], a["scale"], a["M"], a["D"], a["G"],
                                 a["eps"], a["qf"], a["sf"], a["layout"], a["rounding"], act, res,
                                 a["stream"])


BF16, F16, F32 = 0, 1, 2


@pytest.mark.parametrize("act,res,kw,status", [
    (BF16, F16, {}, 5), (F32, BF16, {}, 5), (F32, F16, {}, 5), (F16, BF16, {}, 5),
    (3, F32, {}, 5), (F16, -1, {}, 5),
    (F16, F16, dict(x=None), 1), (BF16, F32, dict(gamma=None), 1),
    (BF16, BF16, dict(x=None), 1), (BF16, BF16, dict(G=32), 3),   # the bf16 pair is fagq_launch
    (F16, F32, dict(D=4000), 2), (F32, F32, dict(eps=-1.0), 6),
    (F16, F32, dict(residual=ctypes.c_void_p(BASE + 0x1_0000_0008)), 4),
    (F32, F32, dict(gamma=ctypes.c_void_p(BASE + 0x2_0000_0004)), 4),
    # residual_out may be exactly residual, or x only when x has the residual's size
    (F16, F32, dict(residual_out=fake(0)), 9),
    (BF16, F32, dict(residual_out=ctypes.c_void_p(BASE + 0x1_0000_0000 + 0x100)), 9),
    # fp32 x spans M * D * 4 = 128 KiB: codes 64 KiB past it overlap (bf16 x would not)
    (F32, F32, dict(q=ctypes.c_void_p(BASE + 0x10000)), 9),
    (F16, F32, dict(norm_out=ctypes.c_void_p(BASE + 0x1_0000_0000 + 0x10000)), 9),
    (F16, F16, dict(M=0), 0), (F32, F32, dict(M=0), 0), (BF16, F32, dict(M=0), 0),
])
def test_typed_launch_validation(lib, act, res, kw, status):
    assert call_typed(lib, act, res, **kw) == status


def test_typed_dtype_errors_are_worded(pkg):
    # The Python checks (reached for every argument the fast path rejects)
    # name the tensor and the type it must have.
    from fagq_mi355x import ops
    M, D = 2, 256
    kw = dict(x_q=torch.empty(M, D, dtype=torch.int8), x_scale=torch.empty(M, 2), group_size=128,
              rounding=None)
    h, f, b = torch.float16, torch.float32, torch.bfloat16
    def explain(x, r, g, ro, norm=None):
        ops._explain(torch.empty(M, D, dtype=x), torch.empty(M, D, dtype=r),
                     torch.empty(D, dtype=g), torch.empty(M, D, dtype=ro),
                     None if norm is None else torch.empty(M, D, dtype=norm), **kw)
    with pytest.raises(TypeError, match="unsupported"):
        explain(h, b, h, b)
    with pytest.raises(TypeError, match="unsupported"):
        explain(f, h, f, h)
    with pytest.raises(TypeError, match="gamma must be float16"):
        explain(h, f, f, f)
    with pytest.raises(TypeError, match="residual_out must be float32"):
        explain(b, f, b, b)
    with pytest.raises(TypeError, match="norm_out must be bfloat16"):
        explain(b, f, b, f, norm=f)
    with pytest.raises(TypeError, match="x must be"):
        explain(torch.int32, f, f, f)


def test_in_place_residual_is_accepted_by_validation(lib):
    # residual_out == residual passes validation; with M = 0 nothing is launched.
    assert call(lib, residual_out=fake(1), M=0) == 0


def test_mapped_launch_rejects_bad_mappings(lib):
    def mapped(wpr, rpb, remap=1, D=7168, mode=0, lds=0, layout=0):
        return lib.fagq_launch_mapped(fake(0), fake(1), fake(2), fake(3), None, fake(4), fake(5),
                                      8, D, 128, 1e-6, 1, 0, layout, 0, wpr, rpb, mode, remap, lds,
                                      None)
    assert mapped(0, 1) == 5
    assert mapped(17, 1) == 5
    assert mapped(4, 5) == 5          # 20 waves > 16
    assert mapped(1, 1) == 5          # 14 steps in one wave (at most 4)
    assert mapped(7, 1, remap=3) == 5
    assert mapped(7, 1, remap=128) == 5
    assert mapped(7, 1, D=65536) == 7  # D above FAGQ_MAX_D
    assert mapped(7, 1, mode=-1) == 5
    assert mapped(7, 1, mode=3) == 5
    assert mapped(4, 2, mode=2) == 5                   # wide scales: column-major only
    assert mapped(4, 1, mode=2, layout=1) == 5         # wide scales: 2 or 4 rows
    assert mapped(4, 3, mode=2, layout=1) == 5
    assert mapped(8, 1, D=16384, mode=1) == 5          # 32 steps of gamma > 16 in LDS
    assert mapped(7, 1, lds=-1) == 5
    assert mapped(7, 1, lds=65537) == 5


def test_diag_validation(lib, probe_lib):
    assert lib.fagq_diag_encode(None, fake(1), 8, 1, 0, 1, None) == 1
    assert lib.fagq_diag_encode(fake(0), fake(1), 9, 1, 0, 1, None) == 2
    assert lib.fagq_diag_encode(fake(0), fake(1), 8, 1, 1, 1, None) == 5
    assert lib.fagq_diag_encode(fake(0), fake(1), 8, 1, 0, 2, None) == 5
    assert lib.fagq_diag_encode(fake(0), fake(1), 0, 1, 0, 0, None) == 0
    assert probe_lib.fagq_diag_copy(fake(0), fake(1), 15, None) == 2
    assert probe_lib.fagq_diag_copy(None, fake(1), 16, None) == 1
    assert probe_lib.fagq_diag_copy(fake(0), fake(1), 0, None) == 0
    assert probe_lib.fagq_diag_stream(fake(0), fake(1), 16, 4, None) == 5
    assert probe_lib.fagq_diag_stream(fake(0), fake(1), 16, 3, None) == 2   # opmix: bytes % 32
    assert probe_lib.fagq_diag_stream(None, fake(1), 16, 1, None) == 1     # read needs src
    assert probe_lib.fagq_diag_stream(fake(0), None, 16, 2, None) == 1
    assert probe_lib.fagq_diag_stream(None, fake(1), 0, 2, None) == 0      # write: src may be NULL
    assert probe_lib.fagq_diag_stream(fake(0), ctypes.c_void_p(BASE + 8), 16, 0, None) == 4
    assert probe_lib.fagq_diag_mfma_peak(None, 1, 1, None) == 1
    assert probe_lib.fagq_diag_mfma_peak(fake(0), 0, 1, None) == 2
    assert probe_lib.fagq_diag_mfma_peak(fake(0), 1, 0, None) == 2
    assert probe_lib.fagq_diag_mfma_rate(fake(0), 1, 1, 2, None) == 5
    assert probe_lib.fagq_diag_mfma_rate(None, 1, 1, 1, None) == 1
    assert probe_lib.fagq_diag_mfma_peak(fake(0), (1 << 20) + 1, 1, None) == 7
    assert probe_lib.fagq_diag_mfma_peak(ctypes.c_void_p(BASE + 2), 1, 1, None) == 4
    assert probe_lib.fagq_diag_lds_read(None, 1, 1, 0, None) == 1
    assert probe_lib.fagq_diag_lds_read(fake(0), 1, 1, 6, None) == 5
    assert probe_lib.fagq_diag_lds_read(fake(0), 1, 1, -1, None) == 5
    assert probe_lib.fagq_diag_lds_read(fake(0), 0, 1, 0, None) == 2
    assert probe_lib.fagq_diag_lds_read(fake(0), 1, 0, 0, None) == 2
    assert probe_lib.fagq_diag_lds_read(fake(0), 1, (1 << 20) + 1, 0, None) == 7
    assert probe_lib.fagq_diag_lds_read(ctypes.c_void_p(BASE + 8), 1, 1, 0, None) == 4


# ----------------------------------------------------------------- Python layer

def cpu_args(M=4, D=512, qdt=torch.float8_e4m3fn):
    x = torch.zeros(M, D, dtype=torch.bfloat16)
    return dict(x=x, residual=x.clone(), gamma=torch.ones(D, dtype=torch.bfloat16),
                residual_out=x.clone(), norm_out=None, x_q=torch.empty(M, D, dtype=qdt),
                x_scale=torch.empty(M, D // 128), eps=1e-6, group_size=128)


def test_cpu_tensors_are_rejected(pkg):
    with pytest.raises(ValueError, match="GPU"):
        pkg.fused_add_rmsnorm_group_quant(**cpu_args())


def test_cpython_binding_is_built_and_bound(pkg):
    # The per-call binding (csrc/fagq_py.cpp) loads, is bound to this process's
    # libfagq.so, and hands every argument it does not accept back to the
    # Python checks (status ARG_ERROR) instead of raising or launching.
    from fagq_mi355x import _fagq_py, _lib
    fast = _lib.fast_launch()
    assert fast is _fagq_py.launch and _fagq_py.ARG_ERROR == _lib.FAST_ARG_ERROR
    a = cpu_args()
    args = [a["x"], a["residual"], a["gamma"], a["residual_out"], None, a["x_q"], a["x_scale"],
            1e-6, 128, -1, 0]
    assert fast(*args) == _lib.FAST_ARG_ERROR          # CPU tensors
    bad = list(args)
    bad[8] = 128.0                                     # a float group size
    assert fast(*bad) == _lib.FAST_ARG_ERROR
    bad = list(args)
    bad[0] = [0.0] * 4                                 # not a tensor
    assert fast(*bad) == _lib.FAST_ARG_ERROR
    with pytest.raises(TypeError):
        fast(*args[:10])
    with pytest.raises(ValueError):
        _fagq_py.bind(0, 0)
    with pytest.raises(TypeError):
        _fagq_py.bind(0)


def test_format_inference(pkg):
    from fagq_mi355x import _lib, ops
    assert ops._q_format(torch.empty(1, dtype=torch.int8)) == _lib.Q_INT8
    assert ops._q_format(torch.empty(1, dtype=torch.float8_e4m3fn)) == _lib.Q_FP8_E4M3FN
    with pytest.raises(TypeError):
        ops._q_format(torch.empty(1, dtype=torch.uint8))
    assert ops._scale_format(torch.empty(1)) == _lib.SCALE_F32
    assert ops._scale_format(torch.empty(1, dtype=torch.uint8)) == _lib.SCALE_UE8M0
    with pytest.raises(TypeError):
        ops._scale_format(torch.empty(1, dtype=torch.float16))
    row = pkg.empty_scales(6, 4)
    col = pkg.empty_scales(6, 4, col_major=True)
    assert ops._scale_layout(row, 6, 4) == _lib.LAYOUT_ROW_MAJOR
    assert ops._scale_layout(col, 6, 4) == _lib.LAYOUT_COL_MAJOR
    assert col.shape == (6, 4) and col.stride() == (1, 6)
    with pytest.raises(ValueError):
        ops._scale_layout(torch.empty(6, 8)[:, ::2], 6, 4)
    with pytest.raises(ValueError):
        ops._scale_layout(row, 6, 5)
    # The reference's int8 cast truncates; fp8 rounds to nearest even only.
    assert ops._rounding(None, _lib.Q_INT8) == _lib.ROUND_TRUNC
    assert ops._rounding("rne", _lib.Q_INT8) == _lib.ROUND_RNE
    assert ops._rounding(None, _lib.Q_FP8_E4M3FN) == _lib.ROUND_RNE
    with pytest.raises(ValueError):
        ops._rounding("trunc", _lib.Q_FP8_E4M3FN)
    with pytest.raises(ValueError):
        ops._rounding("floor", _lib.Q_INT8)


def test_status_errors_name_the_code(pkg):
    from fagq_mi355x import _lib
    err = _lib.FagqError(9)
    assert "FAGQ_E_ALIAS" in str(err) and err.status == 9
    with pytest.raises(_lib.FagqError):
        _lib.check(3)
    _lib.check(0)


# ----------------------------------------------------------------- GEMM consumer

def gemm_call(lib, **kw):
    a = dict(a=fake(0), sa=fake(1), b=fake(2), sb=fake(3), c=fake(4), M=256, N=256, K=1024,
             asf=0, asl=1, bsf=0)
    a.update(kw)
    return lib.fagq_gemm_launch(a["a"], a["sa"], a["b"], a["sb"], a["c"], a["M"], a["N"], a["K"],
                                a["asf"], a["asl"], a["bsf"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(a=None), 1), (dict(sa=None), 1), (dict(b=None), 1), (dict(sb=None), 1), (dict(c=None), 1),
    (dict(asf=2), 5), (dict(bsf=-1), 5), (dict(asl=2), 5),
    (dict(K=1000), 2), (dict(K=0), 2), (dict(N=100), 2), (dict(N=0), 2), (dict(M=-1), 2),
    (dict(K=1 << 24), 7), (dict(N=1 << 23), 7),
    (dict(a=ctypes.c_void_p(BASE + 8)), 4), (dict(c=ctypes.c_void_p(BASE + 0x4_0000_0008)), 4),
    (dict(sa=ctypes.c_void_p(BASE + 0x1_0000_0002)), 4),
    (dict(c=fake(0)), 9), (dict(c=fake(3)), 9),
    (dict(M=0), 0),
])
def test_gemm_validation(lib, kw, status):
    assert gemm_call(lib, **kw) == status


def test_gemm_ue8m0_scales_need_no_alignment(lib):
    # M = 0 so that nothing is launched after validation.
    odd = ctypes.c_void_p(BASE + 0x1_0000_0003)
    assert gemm_call(lib, sa=odd, asf=1, M=0) == 0
    assert gemm_call(lib, sa=odd, asf=0, M=0) == 4


def test_gemm_route(pkg):
    r = pkg.gemm_route(16384, 4096, 7168)
    assert (r["block_m"], r["block_n"], r["block_threads"]) == (256, 256, 512)
    assert r["grid_blocks"] == 64 * 16
    # N = 2112: 11 tiles of 192 columns (704 workgroups, 3 rounds of 256 CUs
    # at 3/4 of the width) against 9 of 256 (576, 3 rounds at full width)
    r = pkg.gemm_route(16384, 2112, 7168)
    assert (r["block_n"], r["grid_blocks"]) == (192, 64 * 11)
    # one round either way: the narrower tile
    assert (pkg.gemm_route(1, 16, 128)["block_n"], pkg.gemm_route(1, 16, 128)["grid_blocks"]) == (192, 1)
    # 6 rounds of 192 (22 tiles per row panel) against 4 of 256
    assert pkg.gemm_route(16384, 4096, 128)["block_n"] == 256
    with pytest.raises(pkg.FagqError):
        pkg.gemm_route(16, 16, 100)


def test_gemm_mapped_validation(lib):
    def mapped(bn, **kw):
        a = dict(a=fake(0), sa=fake(1), b=fake(2), sb=fake(3), c=fake(4), M=0, N=256, K=1024)
        a.update(kw)
        return lib.fagq_gemm_launch_mapped(a["a"], a["sa"], a["b"], a["sb"], a["c"], a["M"], a["N"],
                                           a["K"], 0, 1, 0, bn, None)
    for bn in (0, 192, 256):
        assert mapped(bn) == 0                      # M = 0: validated, nothing launched
    for bn in (-1, 128, 320):
        assert mapped(bn) == 5
    assert mapped(192, K=1000) == 2


def test_gemm_workloads(pkg):
    from fagq_mi355x.workloads import GEMM_CONFIGS, GemmWorkload, make_gemm_inputs
    w = GemmWorkload("t", 300, 272, 512, "f32", "ue8m0", seed=3)
    a_q, a_s, b_q, b_s = make_gemm_inputs(w)
    assert a_q.shape == (300, 512) and a_q.dtype == torch.float8_e4m3fn
    assert a_s.shape == (4, 300) and a_s.dtype == torch.float32
    assert b_q.shape == (272, 512) and b_s.shape == (3, 4) and b_s.dtype == torch.uint8
    again = make_gemm_inputs(w)
    assert torch.equal(again[0].view(torch.uint8), a_q.view(torch.uint8))
    assert GEMM_CONFIGS["gemm_dsv3_16384x4096x7168"].flops() == 2 * 16384 * 4096 * 7168


# --------------------------------------------------------- DSA top-k transform

def dsa_call(lib, **kw):
    a = dict(s=fake(0), sd=0, pt=fake(1), qp=fake(2), kv=fake(3), idx=0, ob=fake(4), op=fake(5),
             B=2, H=4, Q=8, NB=1024, bs=64, k=128)
    a.update(kw)
    return lib.fagq_dsa_topk_launch(a["s"], a["sd"], a["pt"], a["qp"], a["kv"], a["idx"], a["ob"],
                                    a["op"], a["B"], a["H"], a["Q"], a["NB"], a["bs"], a["k"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(s=None), 1), (dict(pt=None), 1), (dict(qp=None), 1), (dict(kv=None), 1),
    (dict(ob=None), 1), (dict(op=None), 1),
    (dict(sd=2), 5), (dict(idx=-1), 5),
    (dict(B=-1), 2), (dict(NB=0), 2), (dict(bs=0), 2), (dict(k=0), 2),
    (dict(NB=(1 << 28) + 1), 7), (dict(k=1025), 7), (dict(bs=1 << 31), 7),
    (dict(H=65536), 7), (dict(B=65536), 7),
    (dict(Q=1 << 26), 7),                          # Q x 64 work-items (1 wave) reach 2^32
    (dict(Q=1 << 22, NB=16384, B=1, H=1), 7),      # Q x 64 x 16 waves reach 2^32
    (dict(Q=1 << 29), 7),                          # B x H x Q >= 2^31
    (dict(s=ctypes.c_void_p(BASE + 2)), 4), (dict(s=ctypes.c_void_p(BASE + 1), sd=1), 4),
    (dict(qp=ctypes.c_void_p(BASE + 0x2_0000_0004), idx=1), 4),
    (dict(op=fake(4)), 9), (dict(op=ctypes.c_void_p(BASE + 0x4_0000_0100)), 9),
    (dict(Q=0), 0),
])
def test_dsa_validation(lib, kw, status):
    assert dsa_call(lib, **kw) == status


# ------------------------------------------------------------ MLA backward (Task 03)

def mla_call(lib, **kw):
    a = dict(q=fake(0), c=fake(1), o=fake(2), do=fake(3), lse=fake(4), dq=fake(5), dc=fake(6),
             ws=fake(7), wsb=1 << 30, B=1, H=4, S=256, D=512, scale=0.05, dqt=0, dct=0)
    a.update(kw)
    return lib.fagq_mla_bwd_launch(a["q"], a["c"], a["o"], a["do"], a["lse"], a["dq"], a["dc"], a["ws"],
                                   a["wsb"], a["B"], a["H"], a["S"], a["D"], a["scale"], a["dqt"],
                                   a["dct"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(q=None), 1), (dict(lse=None), 1), (dict(dc=None), 1), (dict(ws=None), 1),
    (dict(dqt=2), 5), (dict(dct=-1), 5),
    (dict(B=-1), 2), (dict(H=0), 2), (dict(S=0), 2), (dict(D=96), 2), (dict(D=32), 2),
    (dict(scale=float("nan")), 2), (dict(wsb=1000), 2),
    (dict(B=65536), 7), (dict(H=65536, S=64), 7), (dict(H=64, S=1 << 15), 7),
    (dict(H=1, S=1 << 16, D=1 << 14), 7),
    (dict(q=ctypes.c_void_p(BASE + 8)), 4), (dict(lse=ctypes.c_void_p(BASE + 0x4_0000_0002)), 4),
    (dict(ws=ctypes.c_void_p(BASE + 0x7_0000_0004)), 4),
    (dict(dq=fake(0)), 9), (dict(dc=fake(3)), 9), (dict(ws=fake(5)), 9),
    (dict(dc=ctypes.c_void_p(BASE + 0x5_0000_0100)), 9),
    (dict(B=0), 0),
])
def test_mla_validation(lib, kw, status):
    assert mla_call(lib, **kw) == status


def test_mla_workspace_size(lib):
    # head sums [B, S, D] plus the totals of 64-row blocks
    assert lib.fagq_mla_bwd_workspace_bytes(2, 4096, 512) == 2 * (4096 + 64) * 512 * 4
    # small grids split the heads into up to 8 groups, one partial plane each;
    # 16-row blocks
    assert lib.fagq_mla_bwd_workspace_bytes(1, 65, 64) == (8 * 65 + 5) * 64 * 4
    assert lib.fagq_mla_bwd_workspace_bytes(-1, 1, 64) == -1
    # D above 512 runs in 512-wide column slices: the workspace holds one slice
    assert lib.fagq_mla_bwd_workspace_bytes(2, 4096, 1024) == 2 * (4096 + 64) * 512 * 4
    assert lib.fagq_mla_bwd_workspace_bytes(2, 4096, 576) == 2 * (4096 + 64) * 512 * 4


def test_mla_workloads(pkg):
    from fagq_mi355x.workloads import MLA_CONFIGS, MLA_HEADLINE
    w = MLA_CONFIGS[MLA_HEADLINE]
    assert (w.B, w.H, w.S, w.D) == (2, 64, 4096, 512)
    n = 2 * 64 * 4096 * 512
    assert w.algorithmic_bytes() >= 4 * n
