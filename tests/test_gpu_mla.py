"""GPU parity of the Task 03 operator (fagq_mla_bwd_launch) against the CPU
oracle (oracle/mla_bwd_oracle.c).

Bars:
* dq rows >= 16: bit-exact (fp32(do) * sm_scale, then the output cast);
* dq rows < 16 (exact rows): |gpu - oracle| <= 2^-7 sum_j |dS_ij| |c_jd| +
  2^-15 x (the sensitivity of dq to dp - delta) (+ half a bf16 ulp for a bf16
  dq): the kernel accumulates in fp32, so dp - delta, which cancels when out
  is close to c, carries fp32 rounding, and P or dS may round to the
  neighbouring bf16 value where the oracle's float64 value sits near a
  rounding boundary;
* dc: |gpu - oracle| <= 2^-16 sum_{i >= j} sum_h |do[h, i]| / (i + 1)
  (+ half a bf16 ulp for a bf16 dc): fp32 sums in another order.
At the full reference size the oracle runs on the exact rows only; dq rows
>= 16 are checked bit-exact against fp32(do) * sm_scale, and dc against a
float64 reverse scan of the head sums.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import note

pytestmark = pytest.mark.gpu


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint16).numpy()


def as_bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def run_gpu(pkg, dev, q, c, out, do, lse, scale, grad_dtype, dc_dtype=None):
    B, H, S, D = q.shape
    dq = torch.full((B, H, S, D), float("nan"), dtype=grad_dtype, device=dev)
    dc = torch.full((B, S, D), float("nan"), dtype=dc_dtype or grad_dtype, device=dev)
    pkg.mla_bwd_nope_dkdv(q.to(dev), c.to(dev), out.to(dev), do.to(dev), lse.to(dev), dq, dc, scale)
    torch.cuda.synchronize()
    return dq, dc


def check_exact_rows(dq_gpu, dq_ref, bound, bf16_out, label):
    E, D = bound.shape[3], bound.shape[4]
    g = dq_gpu[:, :, :E].float().cpu().numpy().astype(np.float64)
    # bf16 steps of P or dS, plus fp32 accumulation of the D-term dot
    # products behind dp - delta (D x 2^-24 of their magnitude, at least
    # 512 x 2^-24)
    tol = 2.0 ** -7 * bound[0] + max(D, 512) * 2.0 ** -24 * bound[1] + 1e-7
    if bf16_out:
        tol = tol + 2.0 ** -8 * np.abs(dq_ref[:, :, :E])
    err = np.abs(g - dq_ref[:, :, :E])
    assert np.isfinite(g).all() and (err <= tol).all(), \
        f"{label}: exact rows off by {float((err - tol).max())} over tolerance"


def case(pkg, dev, B, H, S, D, grad_dtype, dc_dtype=None, seed=0):
    from fagq_mi355x.workloads import MlaWorkload, make_mla_inputs
    w = MlaWorkload("t", B, H, S, D, grad_dtype, seed)
    q, c, out, do, lse = make_mla_inputs(w)
    label = f"B{B} H{H} S{S} D{D} dq {grad_dtype} dc {dc_dtype or grad_dtype}"
    note(f"mla {label}")
    dq, dc = run_gpu(pkg, dev, q, c, out, do, lse, w.sm_scale, grad_dtype, dc_dtype)
    rdq, rdc, bound = oracle.mla_bwd(bits(q), bits(c), bits(out), bits(do), lse.numpy(), w.sm_scale)
    E = w.exact_rows
    # rows >= E: bit-exact
    want = rdq[:, :, E:].astype(np.float32)
    got = dq[:, :, E:].float().cpu().numpy()
    if grad_dtype == torch.bfloat16:
        want = as_bf16(want)
    assert np.array_equal(got, want), f"{label}: dq rows >= {E} not bit-exact"
    check_exact_rows(dq, rdq, bound, grad_dtype == torch.bfloat16, label)
    # dc
    absdo = np.abs(do.float().numpy()).sum(1) / np.arange(1, S + 1)[None, :, None]
    scale_ref = np.flip(np.cumsum(np.flip(absdo, 1), 1), 1)
    tol = 2.0 ** -16 * scale_ref + 1e-7
    if (dc_dtype or grad_dtype) == torch.bfloat16:
        tol = tol + 2.0 ** -8 * np.abs(rdc)
    g = dc.float().cpu().numpy().astype(np.float64)
    err = np.abs(g - rdc)
    assert np.isfinite(g).all() and (err <= tol).all(), \
        f"{label}: dc off by {float((err - tol).max())} over tolerance"


# Short sequences split the heads into several partial head-sum planes and
# their scan blocks into column slices (S = 256, 512); 769, 1024, 1025 and 2048
# cover block counts that do not divide the rows evenly and fewer planes.
@pytest.mark.parametrize("B,H,S,D", [(1, 4, 64, 512), (2, 3, 100, 64), (1, 2, 10, 128),
                                     (1, 8, 257, 256), (2, 64, 256, 512), (2, 64, 512, 512),
                                     (1, 1, 1, 64), (1, 4, 1024, 128), (1, 4, 1025, 128),
                                     (2, 16, 2048, 64), (2, 8, 769, 512)])
@pytest.mark.parametrize("grad", [torch.float32, torch.bfloat16])
def test_mla_matches_oracle(pkg, gpu, B, H, S, D, grad):
    case(pkg, gpu, B, H, S, D, grad)


@pytest.mark.parametrize("B,H,S,D", [(1, 5, 33, 192), (3, 9, 70, 320), (1, 13, 17, 448),
                                     (1, 7, 129, 384)])
@pytest.mark.parametrize("dq_dtype", [torch.bfloat16, torch.float32])
def test_mla_uneven_head_groups(pkg, gpu, B, H, S, D, dq_dtype):
    # short sequences split the heads into 3, 5, 7 and 4 groups of partial
    # head sums; D not a power of two leaves some scan threads idle, and with
    # fp32 dq the dO pass splits each row into two halves of D / 2
    case(pkg, gpu, B, H, S, D, dq_dtype, torch.float32, seed=B + H + S)


@pytest.mark.parametrize("B,H,S,D", [(1, 4, 40, 576), (2, 3, 10, 1024), (1, 6, 100, 640),
                                     (1, 2, 300, 1152), (2, 64, 256, 1024)])
@pytest.mark.parametrize("dq_dtype", [torch.bfloat16, torch.float32])
def test_mla_column_slices(pkg, gpu, B, H, S, D, dq_dtype):
    # D above 512 runs in 512-wide column slices (the last one 64, 512, 128,
    # 128 and 512 wide): the exact rows stage their rows in chunks and the
    # other kernels run once per slice; the last case's slices each split the
    # heads into 8 partial planes and the block totals into 4 column slices
    case(pkg, gpu, B, H, S, D, dq_dtype, seed=D + S)


def test_mla_mixed_output_dtypes(pkg, gpu):
    case(pkg, gpu, 1, 4, 300, 512, torch.float32, torch.bfloat16, seed=3)
    case(pkg, gpu, 1, 4, 300, 512, torch.bfloat16, torch.float32, seed=4)


@pytest.mark.parametrize("name", ["mla_b2h64s4096d512", "mla_b2h64s4096d512_f32grad"])
def test_mla_reference_workload_full_size(pkg, gpu, name):
    from fagq_mi355x.workloads import MLA_CONFIGS, make_mla_inputs
    w = MLA_CONFIGS[name]
    note(f"mla full size {name}")
    q, c, out, do, lse = make_mla_inputs(w, device=gpu)
    B, H, S, D, E = w.B, w.H, w.S, w.D, w.exact_rows
    dq = torch.empty(B, H, S, D, dtype=w.grad_dtype, device=gpu)
    dc = torch.empty(B, S, D, dtype=w.grad_dtype, device=gpu)
    pkg.mla_bwd_nope_dkdv(q, c, out, do, lse, dq, dc, w.sm_scale)
    torch.cuda.synchronize()
    for b in range(B):                                  # rows >= E, bit-exact, per batch
        want = (do[b, :, E:].float() * w.sm_scale).to(w.grad_dtype)
        assert torch.equal(dq[b, :, E:], want), f"{name}: dq rows >= {E} of batch {b}"
    # exact rows: the oracle on rows 0..E-1 (they depend on nothing past row E-1)
    rdq, _, bound = oracle.mla_bwd(bits(q[:, :, :E]), bits(c[:, :E]), bits(out[:, :, :E]),
                                   bits(do[:, :, :E]), lse[:, :, :E].cpu().numpy(), w.sm_scale)
    check_exact_rows(dq, rdq, bound, w.grad_dtype == torch.bfloat16, name)
    # dc against a float64 reverse scan of the head sums
    hs = torch.zeros(B, S, D, dtype=torch.float64, device=gpu)
    for h in range(H):
        hs += do[:, h].double()
    hs /= torch.arange(1, S + 1, device=gpu, dtype=torch.float64)[None, :, None]
    ref = hs.flip(1).cumsum(1).flip(1)
    ab = torch.zeros(B, S, D, dtype=torch.float64, device=gpu)
    for h in range(H):
        ab += do[:, h].double().abs()
    ab /= torch.arange(1, S + 1, device=gpu, dtype=torch.float64)[None, :, None]
    tol = 2.0 ** -16 * ab.flip(1).cumsum(1).flip(1) + 1e-7
    if w.grad_dtype == torch.bfloat16:
        tol += 2.0 ** -8 * ref.abs()
    err = (dc.double() - ref).abs()
    assert bool(torch.isfinite(dc).all()) and bool((err <= tol).all()), \
        f"{name}: dc off by {float((err - tol).max())} over tolerance"


def test_mla_python_errors(pkg, gpu):
    B, H, S, D = 1, 2, 32, 64
    q = torch.zeros(B, H, S, D, dtype=torch.bfloat16, device=gpu)
    c = torch.zeros(B, S, D, dtype=torch.bfloat16, device=gpu)
    lse = torch.zeros(B, H, S, device=gpu)
    dq = torch.empty(B, H, S, D, device=gpu)
    dc = torch.empty(B, S, D, device=gpu)
    with pytest.raises(ValueError):
        pkg.mla_bwd_nope_dkdv(q.float(), c, q, q, lse, dq, dc, 0.1)
    with pytest.raises(ValueError):
        pkg.mla_bwd_nope_dkdv(q, c, q, q, lse, dq, dc[:, :-1], 0.1)
    with pytest.raises(ValueError):
        pkg.mla_bwd_nope_dkdv(q, c, q, q, lse, dq, dc, 0.1,
                              workspace=torch.empty(16, dtype=torch.uint8, device=gpu))
    from fagq_mi355x import FagqError
    with pytest.raises(FagqError):                    # D % 64 != 0
        z = torch.zeros(B, H, S, 96, dtype=torch.bfloat16, device=gpu)
        pkg.mla_bwd_nope_dkdv(z, torch.zeros(B, S, 96, dtype=torch.bfloat16, device=gpu), z, z, lse,
                              torch.empty(B, H, S, 96, device=gpu), torch.empty(B, S, 96, device=gpu),
                              0.1)
