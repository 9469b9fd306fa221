"""GPU parity of the typed form (fagq_launch_typed): fp16 activations and an
fp32 residual stream, as the reference's dtype-generic kernels take them
(task01.py:88-94 convert loads to fp32, :91 and :118 round stores to the
destination's type).  Checked against the oracle's orc_fagq_typed on the same
inputs, through the reference-signature Python operator; residual_out and
norm_out are compared as bit patterns (so -0 and +0 differ), scales and codes
bit for bit."""
import numpy as np
import pytest
import torch

import oracle
from oracle.compare import compare
from tests.gpu_util import FMTS, note

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: oracle.DT_BF16, torch.float16: oracle.DT_F16, torch.float32: oracle.DT_F32}
PAIRS = [(torch.float16, torch.float16), (torch.bfloat16, torch.float32),
         (torch.float16, torch.float32), (torch.float32, torch.float32)]


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous().cpu()
    return t.view(torch.int32).numpy().view(np.uint32) if t.dtype == torch.float32 else \
        t.view(torch.int16).numpy().view(np.uint16)


def store(t: torch.Tensor) -> np.ndarray:
    """The oracle's storage of a CPU tensor: bf16/fp16 as uint16 bits, fp32 as float32."""
    t = t.contiguous()
    return t.numpy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16)


def make(M, D, at, rt, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (scale * torch.randn(M, D, generator=g)).to(at)
    r = (scale * torch.randn(M, D, generator=g)).to(rt)
    w = (1.0 + 0.1 * torch.randn(D, generator=g)).to(at)
    return x, r, w


def run(pkg, dev, x, r, w, G=128, fmt="fp8", ue8m0=False, col=False, with_norm=False,
        inplace=False, eps=1e-6, label=""):
    M, D = x.shape
    note(f"case typed {label}: M={M} D={D} x={x.dtype} residual={r.dtype} G={G} {fmt} "
         f"ue8m0={ue8m0} col={col} norm={with_norm} inplace={inplace}")
    qdt, rnd, qf, orc_rnd = FMTS[fmt]
    xd, rd, wd = x.to(dev), r.to(dev), w.to(dev)
    ro = rd if inplace else torch.empty_like(rd)
    q = torch.empty((M, D), dtype=qdt, device=dev)
    sc = pkg.empty_scales(M, D // G, ue8m0=ue8m0, col_major=col, device=dev)
    norm = torch.empty_like(xd) if with_norm else None
    pkg.fused_add_rmsnorm_group_quant(xd, rd, wd, ro, norm, q, sc, eps, G,
                                      rounding=rnd if qdt == torch.int8 else None)
    torch.cuda.synchronize(dev)
    ref = oracle.fagq_typed(store(x), store(r), store(w), eps, G, DT[x.dtype], DT[r.dtype], qf,
                            oracle.S_UE8M0 if ue8m0 else oracle.S_F32,
                            oracle.L_COL if col else oracle.L_ROW, orc_rnd, with_norm)
    as_bits = lambda a: a.view(np.uint32) if a.dtype == np.float32 else a
    refb = {"residual_out": as_bits(ref["residual_out"]), "q": ref["q"], "scale": ref["scale"]}
    phys = sc.t() if col else sc
    gpub = {"residual_out": bits(ro), "q": q.cpu().view(torch.uint8).numpy(),
            "scale": np.ascontiguousarray(phys.cpu().numpy())}
    if with_norm:
        refb["norm_out"] = as_bits(ref["norm_out"])
        gpub["norm_out"] = bits(norm)
    st = compare(gpub, refb, fp8=fmt == "fp8", ue8m0=ue8m0, label=label)
    assert st["exact"], st
    return st


# Shapes reaching every steps-per-wave count of the typed route (the families
# with an fp32 tensor): decode rows (M < 1024) take 1-step waves up to
# D = 8192, then ceil(D / 8192) steps; prefill rows take 1 step at 5..8 steps
# per row and 2 otherwise.  fp16 tensors take the bf16 operator's route.
@pytest.mark.parametrize("at,rt", PAIRS)
@pytest.mark.parametrize("M,D", [(7, 4096), (5, 16384), (3, 24576), (2, 32768), (1024, 4096),
                                 (1024, 7168), (33, 1536)])
def test_typed_shapes(pkg, gpu, at, rt, M, D):
    x, r, w = make(M, D, at, rt, seed=D + M)
    run(pkg, gpu, x, r, w, with_norm=True, label=f"shape {M}x{D}")


@pytest.mark.parametrize("at,rt", PAIRS)
@pytest.mark.parametrize("G", [64, 128, 256])
@pytest.mark.parametrize("fmt", ["fp8", "int8_rne", "int8_trunc"])
@pytest.mark.parametrize("ue8m0,col", [(False, False), (True, True), (False, True)])
def test_typed_format_matrix(pkg, gpu, at, rt, G, fmt, ue8m0, col):
    x, r, w = make(37, 3072, at, rt, seed=G, scale=2.0)
    run(pkg, gpu, x, r, w, G, fmt, ue8m0, col, with_norm=(G == 128), label="format")


# fp16 tensors run the bf16 operator's kernels with fp16 elements and its
# route, row-group modes included: 2 rows per workgroup sharing gamma, with the
# column-major scales of both rows stored together (mode 2), and independent
# rows (mode 0); M = 2049 leaves a last workgroup with one row.
@pytest.mark.parametrize("M,D,ue8m0,col,mode", [(2048, 7168, False, True, 2),
                                                (2049, 7168, True, True, 2),
                                                (2048, 7168, False, False, 0),
                                                (4096, 4096, True, True, 0)])
def test_f16_route_modes(pkg, gpu, M, D, ue8m0, col, mode):
    from fagq_mi355x import _lib
    route = _lib.query_route(M, D, 128, 1 if ue8m0 else 0, 1 if col else 0)
    assert route["row_group_mode"] == mode, route
    x, r, w = make(M, D, torch.float16, torch.float16, seed=M + D)
    run(pkg, gpu, x, r, w, ue8m0=ue8m0, col=col, with_norm=True, label=f"f16 mode {mode}")


@pytest.mark.parametrize("name", ["f16_16384x7168", "bf16_r32_16384x7168"])
def test_typed_workloads_full_size(pkg, gpu, name):
    """The bench's typed workloads at full size (the headline shape and format)."""
    from fagq_mi355x.workloads import TYPED_CONFIGS, make_inputs
    w = TYPED_CONFIGS[name]
    x, r, g = make_inputs(w)
    run(pkg, gpu, x, r, g, w.group_size, "fp8", w.scale_ue8m0, w.scale_col_major, label=name)


@pytest.mark.parametrize("at,rt", PAIRS)
def test_typed_in_place_residual(pkg, gpu, at, rt):
    x, r, w = make(64, 7168, at, rt, seed=3)
    run(pkg, gpu, x, r, w, inplace=True, label="in place")


def test_f16_rounding_edges(pkg, gpu):
    """fp16 residual_out / norm_out at the edges of the format: sums that
    overflow to +-inf (|x + residual| >= 65520 while r stays finite in fp32),
    sums in the subnormal range, and ties between fp16 neighbours; all rounded
    to nearest even as the oracle's encoder (pinned against torch's cast)."""
    M, D = 16, 2048
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M, D, generator=g)
    r = torch.randn(M, D, generator=g)
    x[0, :64] = 60000.0
    r[0, :64] = torch.linspace(5000.0, 6000.0, 64)               # sums past 65504
    x[1] = torch.randn(D, generator=g) * 3e-6                     # subnormal sums
    r[1] = torch.randn(D, generator=g) * 3e-6
    x[2, :128] = 1.0
    r[2, :128] = torch.arange(128) * 2.0 ** -11                   # exact ties at 1 + k 2^-11
    x, r = x.half(), r.half()
    w = (1.0 + 0.1 * torch.randn(D, generator=g)).half()
    run(pkg, gpu, x, r, w, with_norm=True, label="f16 edges")
    # fp32 residual stream, fp16 activations: x + residual in fp32, then fp16 norm_out.
    run(pkg, gpu, x, r.float(), w, with_norm=True, label="f16 edges, f32 residual")


def test_typed_bf16_pair_is_the_bf16_operator(pkg, gpu):
    """fagq_launch_typed(BF16, BF16) is fagq_launch: same bits."""
    import ctypes
    from fagq_mi355x import _lib
    M, D = 300, 7168
    x, r, w = make(M, D, torch.bfloat16, torch.bfloat16, seed=9)
    xd, rd, wd = x.to(gpu), r.to(gpu), w.to(gpu)
    outs = []
    L = pkg.load_library()
    for typed in (False, True):
        ro = torch.empty_like(rd)
        q = torch.empty((M, D), dtype=torch.float8_e4m3fn, device=gpu)
        sc = pkg.empty_scales(M, D // 128, col_major=True, device=gpu)
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        args = [p(xd), p(rd), p(wd), p(ro), None, p(q), p(sc), M, D, 128, 1e-6,
                _lib.Q_FP8_E4M3FN, _lib.SCALE_F32, _lib.LAYOUT_COL_MAJOR, _lib.ROUND_RNE]
        st = L.fagq_launch_typed(*args, _lib.DT_BF16, _lib.DT_BF16, None) if typed else \
            L.fagq_launch(*args, None)
        _lib.check(st)
        torch.cuda.synchronize(gpu)
        outs.append((bits(ro), q.cpu().view(torch.uint8).numpy(), sc.t().cpu().numpy()))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def test_typed_python_errors(pkg, gpu):
    M, D = 4, 1024
    x = torch.randn(M, D, device=gpu).half()
    r = torch.randn(M, D, device=gpu).bfloat16()
    w = torch.ones(D, device=gpu).half()
    q = torch.empty(M, D, dtype=torch.float8_e4m3fn, device=gpu)
    sc = torch.empty(M, D // 128, device=gpu)
    with pytest.raises(TypeError, match="unsupported"):         # (fp16, bf16) is not a pair
        pkg.fused_add_rmsnorm_group_quant(x, r, w, torch.empty_like(r), None, q, sc, 1e-6, 128)
    r = r.float()
    with pytest.raises(TypeError, match="gamma"):               # gamma must have x's type
        pkg.fused_add_rmsnorm_group_quant(x, r, w.float(), torch.empty_like(r), None, q, sc, 1e-6,
                                          128)
    with pytest.raises(TypeError, match="residual_out"):        # residual_out: residual's type
        pkg.fused_add_rmsnorm_group_quant(x, r, w, torch.empty_like(x), None, q, sc, 1e-6, 128)
    with pytest.raises(TypeError, match="norm_out"):            # norm_out: x's type
        pkg.fused_add_rmsnorm_group_quant(x, r, w, torch.empty_like(r), torch.empty_like(r), q,
                                          sc, 1e-6, 128)
