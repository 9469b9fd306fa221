"""Seeded random cases on the GPU, each against the CPU oracle at the bar of
the fixed-case parity tests: the operator (bf16 and the typed form), the
multi-input form, DSA top-k, the fp8 GEMM and the MLA backward over shapes,
formats and layouts drawn at random, so that combinations the fixed lists do
not name are exercised too.  The seed of each case is its test id: a failure
names the case to rerun."""
import math
import random

import pytest
import torch

from oracle.compare import compare
from tests.gpu_util import note, run_gpu, run_ref
from tests import test_gpu_dsa as dsa
from tests import test_gpu_gemm as gemm
from tests import test_gpu_mla as mla
from tests import test_gpu_parts as parts
from tests import test_gpu_typed as typed

pytestmark = pytest.mark.gpu

FMT_NAMES = ["fp8", "int8_rne", "int8_trunc"]


def log_uniform(rng: random.Random, lo: int, hi: int) -> int:
    return int(round(math.exp(rng.uniform(math.log(lo), math.log(hi)))))


def shape(rng: random.Random, max_elems: int, max_d: int):
    """(M, D, G): D a multiple of G (64, 128 or 256) up to max_d, M so that M D
    stays under max_elems."""
    G = rng.choice([64, 128, 256])
    D = G * rng.randint(1, max_d // G)
    M = log_uniform(rng, 1, max(1, min(4096, max_elems // D)))
    return M, D, G


@pytest.mark.parametrize("seed", range(200))
def test_random_operator(pkg, gpu, seed):
    rng = random.Random(1000 + seed)
    M, D, G = shape(rng, 6_000_000, 16384)
    fmt = rng.choice(FMT_NAMES)
    ue8m0 = rng.random() < 0.4
    col = rng.random() < 0.6
    with_norm = rng.random() < 0.5
    inplace = rng.random() < 0.3
    scale = 10.0 ** rng.uniform(-3, 3)
    g = torch.Generator().manual_seed(seed)
    x = (scale * torch.randn(M, D, generator=g)).bfloat16()
    r = (scale * torch.randn(M, D, generator=g)).bfloat16()
    if rng.random() < 0.3:      # a few outlier channels
        ch = torch.randint(0, D, (max(1, D // 100),), generator=g)
        x[:, ch] *= 50
    w = (1.0 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    label = (f"random operator {seed}: M={M} D={D} G={G} {fmt} ue8m0={ue8m0} col={col} "
             f"norm={with_norm} inplace={inplace} scale={scale:.3g}")
    note(label)
    got = run_gpu(pkg, gpu, x, r, w, G, fmt, ue8m0, col, with_norm=with_norm, inplace=inplace)
    want = run_ref(x, r, w, G, fmt, ue8m0, col, with_norm=with_norm)
    st = compare(got, want, fp8=fmt == "fp8", ue8m0=ue8m0, label=label)
    assert st["exact"], st


@pytest.mark.parametrize("seed", range(10))
def test_random_operator_large(pkg, gpu, seed):
    """Large grids: M up to 40000, D up to 32768, up to 60 M elements."""
    rng = random.Random(7000 + seed)
    G = rng.choice([64, 128, 256])
    D = G * rng.randint(1, 32768 // G)
    M = log_uniform(rng, 1024, max(1024, min(40000, 60_000_000 // D)))
    fmt = rng.choice(FMT_NAMES)
    ue8m0 = rng.random() < 0.4
    col = rng.random() < 0.6
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, D, generator=g).bfloat16()
    r = torch.randn(M, D, generator=g).bfloat16()
    w = (1.0 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    label = f"random large operator {seed}: M={M} D={D} G={G} {fmt} ue8m0={ue8m0} col={col}"
    note(label)
    got = run_gpu(pkg, gpu, x, r, w, G, fmt, ue8m0, col)
    want = run_ref(x, r, w, G, fmt, ue8m0, col)
    st = compare(got, want, fp8=fmt == "fp8", ue8m0=ue8m0, label=label)
    assert st["exact"], st


@pytest.mark.parametrize("seed", range(80))
def test_random_typed(pkg, gpu, seed):
    rng = random.Random(2000 + seed)
    M, D, G = shape(rng, 3_000_000, 16384)
    at, rt = rng.choice(typed.PAIRS)
    fmt = rng.choice(FMT_NAMES)
    ue8m0 = rng.random() < 0.4
    col = rng.random() < 0.6
    x, r, w = typed.make(M, D, at, rt, seed=seed, scale=10.0 ** rng.uniform(-2, 2))
    typed.run(pkg, gpu, x, r, w, G, fmt, ue8m0, col, with_norm=rng.random() < 0.5,
              inplace=rng.random() < 0.3, label=f"random typed {seed}")


@pytest.mark.parametrize("seed", range(40))
def test_random_parts(pkg, gpu, seed):
    rng = random.Random(3000 + seed)
    nparts = rng.randint(1, 8)
    M, D, G = shape(rng, 2_000_000 // nparts, 16384)
    out = rng.choice([parts.FP8, torch.int8])
    rnd = rng.choice(["rne", "trunc"]) if out == torch.int8 else "rne"
    col, ue = rng.random() < 0.6, rng.random() < 0.4
    label = f"random parts {seed}: P={nparts} M={M} D={D} G={G} {out} col={col} ue8m0={ue} {rnd}"
    note(label)
    p, r, w = parts.inputs(nparts, M, D, seed=seed)
    got = parts.run(pkg, gpu, p, r, w, G, out, col, ue, rnd)
    want = parts.ref(p, r, w, G, out, col, ue, rnd)
    st = compare(got, want, fp8=out == parts.FP8, ue8m0=ue, label=label)
    assert st["exact"], st


TIES = [None, None, None, "round", "heavy", "equal", "outlier", "cluster", "offset", "offset_lin"]


@pytest.mark.parametrize("seed", range(120))
def test_random_dsa(pkg, gpu, seed):
    rng = random.Random(4000 + seed)
    B, H = rng.randint(1, 2), rng.randint(1, 4)
    Q = rng.randint(1, 48)
    NB = log_uniform(rng, 1, 6000)
    bs = rng.choice([1, 7, 16, 64, 128])
    k = log_uniform(rng, 1, 1024)
    dtype = rng.choice([torch.float32, torch.bfloat16])
    idx = rng.choice([torch.int32, torch.int64])
    ties = rng.choice(TIES)
    if ties == "outlier" and NB < 4:       # the helper places the outlier at block 3
        ties = None
    s, pt, pos, kv = dsa.case(seed, B=B, H=H, Q=Q, NB=NB, bs=bs, dtype=dtype, ties=ties, idx=idx)
    dsa.check(pkg, gpu, s, pt, pos, kv, bs, k,
              f"random {seed}: ties={ties} idx={idx}")


@pytest.mark.parametrize("seed", range(40))
def test_random_gemm(pkg, gpu, seed):
    rng = random.Random(5000 + seed)
    N = 16 * rng.randint(1, 256)
    K = 128 * rng.randint(1, 32)
    M = log_uniform(rng, 1, max(1, min(2048, 400_000_000 // (N * K))))
    afmt, bfmt, col = rng.choice(gemm.FORMATS)
    label = f"random gemm {seed}: {M}x{N}x{K} {afmt}/{bfmt} col={col}"
    note(label)
    a_q, a_s, b_q, b_s = gemm.make(M, N, K, afmt, bfmt, col, seed=seed)
    got = gemm.run_gpu(pkg, gpu, a_q, a_s, b_q, b_s, col)
    ref, bound = gemm.run_ref(a_q, a_s, b_q, b_s, col)
    gemm.assert_close(got, ref, bound, K, label)


@pytest.mark.parametrize("seed", range(30))
def test_random_mla(pkg, gpu, seed):
    rng = random.Random(6000 + seed)
    B, H = rng.randint(1, 2), rng.randint(1, 16)
    S = log_uniform(rng, 1, 1200)
    D = 64 * rng.randint(1, 10)
    grad = rng.choice([torch.float32, torch.bfloat16])
    dc = rng.choice([None, torch.float32, torch.bfloat16])
    mla.case(pkg, gpu, B, H, S, D, grad, dc, seed=seed)
