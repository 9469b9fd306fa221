"""GPU parity of the fp8 block-scaled GEMM (fagq_gemm_launch) against the CPU
oracle (oracle/gemm_oracle.c), and its consumption of the quantizer's output.

Tolerance (floating point; the oracle is exact up to double rounding):
  |C_gpu - C_ref| <= 2^-8 |C_ref| + 2 (K/128 + 130) 2^-23 B
where B = sum_kb |s| sum_k |A B| (returned by the oracle): 2^-8 is bf16's
half-ulp, and (K/128 + 130) 2^-23 B bounds any fp32 evaluation of a
128-term block sum, its scaling and the sum over K/128 blocks, even with
truncating additions.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import note

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def rand_fp8(g, shape, lim=448.0):
    v = torch.randn(shape, generator=g) * (lim / 8)
    return v.clamp(-lim, lim).to(FP8)


def rand_scales(g, shape, fmt):
    if fmt == "f32":
        return torch.exp(torch.empty(shape).uniform_(-12, 2, generator=g)).float()
    return torch.randint(100, 140, shape, generator=g, dtype=torch.uint8)


def make(M, N, K, afmt, bfmt, col, seed=0):
    g = torch.Generator().manual_seed(seed)
    kb, nb = K // 128, (N + 127) // 128
    a_q, b_q = rand_fp8(g, (M, K)), rand_fp8(g, (N, K))
    a_s = rand_scales(g, (kb, M) if col else (M, kb), afmt)     # physical layout
    b_s = rand_scales(g, (nb, kb), bfmt)
    return a_q, a_s, b_q, b_s


def run_gpu(pkg, dev, a_q, a_s, b_q, b_s, col):
    a_scale = a_s.to(dev).t() if col else a_s.to(dev)
    out = pkg.fp8_block_scaled_gemm(a_q.to(dev), a_scale, b_q.to(dev), b_s.to(dev))
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def run_ref(a_q, a_s, b_q, b_s, col):
    u8 = lambda t: t.contiguous().view(torch.uint8).numpy()
    return oracle.gemm(u8(a_q), a_s.numpy(), u8(b_q), b_s.numpy(),
                       a_layout=oracle.L_COL if col else oracle.L_ROW)


def assert_close(got, ref, bound, K, label=""):
    tol = 2.0 ** -8 * np.abs(ref) + 2 * (K // 128 + 130) * 2.0 ** -23 * bound
    err = np.abs(got - ref)
    bad = err > tol
    assert np.isfinite(got).all(), label
    assert not bad.any(), (f"{label}: {bad.sum()} of {bad.size} outside tolerance; "
                           f"worst excess {np.max(err - tol):.3g}")


FORMATS = [("f32", "f32", True), ("f32", "f32", False), ("ue8m0", "ue8m0", True),
           ("ue8m0", "f32", True), ("f32", "ue8m0", False)]


@pytest.mark.parametrize("afmt,bfmt,col", FORMATS)
@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (64, 256, 384), (130, 2112, 640),
                                   (300, 272, 1024), (17, 2112, 7168)])
def test_gemm_formats(pkg, gpu, M, N, K, afmt, bfmt, col):
    note(f"gemm M={M} N={N} K={K} a={afmt} b={bfmt} col={col}")
    a_q, a_s, b_q, b_s = make(M, N, K, afmt, bfmt, col, seed=M + N + K)
    got = run_gpu(pkg, gpu, a_q, a_s, b_q, b_s, col)
    ref, bound = run_ref(a_q, a_s, b_q, b_s, col)
    assert_close(got, ref, bound, K, f"{M}x{N}x{K} {afmt}/{bfmt} col={col}")


@pytest.mark.parametrize("afmt,bfmt,col", FORMATS)
@pytest.mark.parametrize("M,N,K", [(300, 2112, 1024), (257, 400, 512), (513, 1536, 256),
                                   (17, 16, 128)])
def test_gemm_tile_widths_agree_bitwise(pkg, gpu, M, N, K, afmt, bfmt, col):
    # 192- and 256-column tiles give the same bits (each output takes the same
    # MFMA and scale sequence); with 192 a wave's 96 columns start at a
    # multiple of 32 mod 128 and may straddle two weight blocks (N = 400,
    # 1536, 2112 all have such waves).  The 192 result is also checked
    # against the oracle.
    import ctypes
    note(f"gemm widths M={M} N={N} K={K} a={afmt} b={bfmt} col={col}")
    a_q, a_s, b_q, b_s = make(M, N, K, afmt, bfmt, col, seed=M + N)
    lib = pkg._lib.load()
    d = [t.to(gpu).contiguous() for t in (a_q, a_s, b_q, b_s)]
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    outs = {}
    for bn in (192, 256):
        c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        st = lib.fagq_gemm_launch_mapped(P(d[0]), P(d[1]), P(d[2]), P(d[3]), P(c), M, N, K,
                                         0 if afmt == "f32" else 1, 1 if col else 0,
                                         0 if bfmt == "f32" else 1, bn,
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert st == 0, st
        torch.cuda.synchronize()
        outs[bn] = c.cpu()
    assert torch.equal(outs[192].view(torch.int16), outs[256].view(torch.int16))
    ref, bound = run_ref(a_q, a_s, b_q, b_s, col)
    assert_close(outs[192].float().numpy(), ref, bound, K, f"BN 192 M={M} N={N}")


@pytest.mark.parametrize("M", [1, 3, 255, 257, 513])
@pytest.mark.parametrize("N", [16, 144, 400])
def test_gemm_ragged_shapes(pkg, gpu, M, N):
    K = 256
    note(f"gemm ragged M={M} N={N} K={K}")
    a_q, a_s, b_q, b_s = make(M, N, K, "f32", "f32", True, seed=M * 7 + N)
    got = run_gpu(pkg, gpu, a_q, a_s, b_q, b_s, True)
    ref, bound = run_ref(a_q, a_s, b_q, b_s, True)
    assert_close(got, ref, bound, K, f"ragged {M}x{N}")


def test_gemm_scale_layouts_agree_bitwise(pkg, gpu):
    M, N, K = 384, 512, 1024
    note(f"gemm layouts M={M} N={N} K={K}")
    a_q, a_s, b_q, b_s = make(M, N, K, "f32", "f32", True, seed=5)
    col = run_gpu(pkg, gpu, a_q, a_s, b_q, b_s, True)
    row = run_gpu(pkg, gpu, a_q, a_s.t().contiguous(), b_q, b_s, False)
    assert np.array_equal(col, row)
    again = run_gpu(pkg, gpu, a_q, a_s, b_q, b_s, True)
    assert np.array_equal(col, again)      # deterministic


def test_gemm_headline_shape_sampled_rows(pkg, gpu):
    """16384 x 4096 x 7168 at full size; 24 rows (edges and random) against the oracle."""
    from fagq_mi355x.workloads import GEMM_CONFIGS, make_gemm_inputs
    w = GEMM_CONFIGS["gemm_dsv3_16384x4096x7168"]
    note(f"gemm full size {w.name}")
    a_q, a_s, b_q, b_s = make_gemm_inputs(w)
    got = run_gpu(pkg, gpu, a_q, a_s, b_q, b_s, True)
    rows = np.unique(np.concatenate([[0, 1, 255, 256, w.M - 1],
                                     np.random.default_rng(0).integers(0, w.M, 19)]))
    ref, bound = run_ref(a_q[rows], a_s[:, rows].contiguous(), b_q, b_s, True)
    assert_close(got[rows], ref, bound, w.K, "headline rows")


@pytest.mark.parametrize("ue8m0", [False, True])
def test_gemm_consumes_quantizer_output(pkg, gpu, ue8m0):
    """Quantize on the GPU (column-major scales, the wire format), multiply, and check
    against the oracle on the same codes and scales, and against the fp32 product of the
    unquantized normalized activations."""
    M, D, N = 512, 7168, 1024
    note(f"gemm after quantizer M={M} K={D} N={N} ue8m0={ue8m0}")
    g = torch.Generator().manual_seed(11)
    x = torch.randn(M, D, generator=g).bfloat16()
    r = torch.randn(M, D, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    b_q = rand_fp8(g, (N, D), lim=64.0)
    b_s = rand_scales(g, (N // 128, D // 128), "ue8m0" if ue8m0 else "f32")
    xd, rd, wd = x.to(gpu), r.to(gpu), w.to(gpu)
    _, q, sc = pkg.fused_add_rmsnorm_group_quant_fn(xd, rd, wd, 1e-6, 128, FP8,
                                                    scale_col_major=True, scale_ue8m0=ue8m0)
    assert sc.stride() == (1, M)
    c = pkg.fp8_block_scaled_gemm(q, sc, b_q.to(gpu), b_s.to(gpu)).float().cpu().numpy()
    q_cpu = q.cpu()
    s_phys = sc.t().contiguous().cpu()
    ref, bound = run_ref(q_cpu, s_phys, b_q, b_s, True)
    assert_close(c, ref, bound, D, "quantizer -> gemm")
    # Against the unquantized activations: fp8 codes carry ~2^-4 relative error.
    rr = x.float() + r.float()
    inv = torch.rsqrt((rr.double() ** 2).mean(1, keepdim=True) + 1e-6).float()
    act = rr * w.float() * inv
    sb = (b_s.float() if not ue8m0 else torch.ldexp(torch.ones(1), b_s.to(torch.int32) - 127))
    B = b_q.float() * sb.repeat_interleave(128, 0).repeat_interleave(128, 1)
    exact = (act.double() @ B.double().T).numpy()
    rel = np.linalg.norm(c - exact) / np.linalg.norm(exact)
    assert rel < 0.05, rel


def test_gemm_python_errors(pkg, gpu):
    a = torch.zeros(4, 256, dtype=FP8, device=gpu)
    s = torch.ones(4, 2, device=gpu)
    b = torch.zeros(128, 256, dtype=FP8, device=gpu)
    bs = torch.ones(1, 2, device=gpu)
    with pytest.raises(TypeError):
        pkg.fp8_block_scaled_gemm(a.view(torch.uint8), s, b, bs)
    with pytest.raises(ValueError):
        pkg.fp8_block_scaled_gemm(a[:, :200], s, b, bs)
    with pytest.raises(ValueError):
        pkg.fp8_block_scaled_gemm(a, s, b, torch.ones(2, 2, device=gpu))
    with pytest.raises(ValueError):
        pkg.fp8_block_scaled_gemm(a, torch.ones(4, 2, device=gpu)[:, :1].expand(4, 2), b, bs)
    out = pkg.fp8_block_scaled_gemm(a, s, b, bs)
    torch.cuda.synchronize()
    assert out.shape == (4, 128) and out.dtype == torch.bfloat16 and not out.float().any()


@pytest.mark.parametrize("col", [True, False])
def test_gemm_copy_offsets_past_2_31(pkg, gpu, col):
    """K = 8,454,144: the operand copies of a 256-row tile start up to 255 K bytes
    (about 2.16e9, past 2^31) into the tile's buffer, so the uint32 offset
    arithmetic (and its range check) is exercised where signed 32-bit offsets
    would overflow.  Only five 128-column blocks are non-zero (the first two, the
    middle one and the last two, in every row, including rows 248..255 whose
    offsets are all past 2^31); every other block multiplies exact zeros, which
    leave an fp32 accumulator unchanged, so the product equals the oracle's on
    the five blocks alone, with the tolerance of that K."""
    M = N = 256
    kb_total = 66048
    K = kb_total * 128
    assert 255 * K > 2 ** 31 and 256 * K < 2 ** 32
    blocks = [0, 1, kb_total // 2, kb_total - 2, kb_total - 1]
    note(f"gemm K={K} (offsets past 2^31) col={col}")
    g = torch.Generator().manual_seed(77)
    a_small, a_s_small, b_small, b_s_small = make(M, N, 128 * len(blocks), "f32", "f32", col, seed=77)
    a_q = torch.zeros((M, K), dtype=torch.uint8, device=gpu)
    b_q = torch.zeros((N, K), dtype=torch.uint8, device=gpu)
    for i, kb in enumerate(blocks):
        a_q[:, kb * 128:(kb + 1) * 128] = a_small[:, i * 128:(i + 1) * 128].view(torch.uint8).to(gpu)
        b_q[:, kb * 128:(kb + 1) * 128] = b_small[:, i * 128:(i + 1) * 128].view(torch.uint8).to(gpu)
    # Scales everywhere (the zero blocks' scales are finite, so they contribute 0).
    a_s_full = torch.exp(torch.empty((kb_total, M) if col else (M, kb_total)).uniform_(-4, 2, generator=g))
    b_s_full = torch.exp(torch.empty(N // 128, kb_total).uniform_(-4, 2, generator=g))
    sel = torch.tensor(blocks)
    if col:
        a_s_full[sel, :] = a_s_small
    else:
        a_s_full[:, sel] = a_s_small
    b_s_full[:, sel] = b_s_small
    a_scale = a_s_full.to(gpu).t() if col else a_s_full.to(gpu)
    c = pkg.fp8_block_scaled_gemm(a_q.view(FP8), a_scale, b_q.view(FP8), b_s_full.to(gpu))
    torch.cuda.synchronize()
    got = c.float().cpu().numpy()
    del a_q, b_q
    ref, bound = run_ref(a_small, a_s_small, b_small, b_s_small, col)
    assert_close(got, ref, bound, 128 * len(blocks), f"K={K} col={col}")
