"""Pins the CPU oracle of the fp8 block-scaled GEMM (oracle/gemm_oracle.c)
before it checks the GPU.

The GEMM has no counterpart in the reference repository (it consumes the
reference operator's output format), so there are no golden vectors.  The
oracle is pinned by:
* its fp8 decoder against torch's float8_e4m3fn cast, on all 256 codes;
* an independent route to the same numbers: dequantize A and B with torch,
  expand the scales to full matrices, and multiply in float64 with numpy
  (this catches a transposed scale layout, a wrong weight-block index, a
  dropped scale or a K-block misalignment);
* known answers (one-hot rows select scaled weight entries; power-of-two
  scales are exact);
* the error bound it returns bounding |C|.
"""
import numpy as np
import pytest
import torch

import oracle

FP8 = torch.float8_e4m3fn


def rand_fp8(rng, shape, lim=448.0):
    v = rng.standard_normal(shape) * (lim / 8)
    v = np.clip(v, -lim, lim).astype(np.float32)
    return torch.from_numpy(v).to(FP8).view(torch.uint8).numpy()


def rand_scales(rng, shape, fmt):
    if fmt == "f32":
        return (np.exp(rng.uniform(-12, 2, size=shape))).astype(np.float32)
    return rng.integers(100, 140, size=shape).astype(np.uint8)


def dequant_ref(a_q, a_scale, b_q, b_scale, a_layout):
    """Independent restatement: (A * sa) @ (B * sb)^T in float64."""
    M, K = a_q.shape
    N = b_q.shape[0]
    A = torch.from_numpy(a_q).view(FP8).to(torch.float64).numpy()
    B = torch.from_numpy(b_q).view(FP8).to(torch.float64).numpy()
    sa = a_scale.T if a_layout == oracle.L_COL else a_scale          # [M, K/128]
    to64 = lambda s: (np.ldexp(1.0, s.astype(np.int64) - 127) if s.dtype == np.uint8
                      else s.astype(np.float64))
    sa, sb = to64(sa), to64(b_scale)
    # fp32 product of the two scales, as the definition states
    s = (sa.astype(np.float32)[:, None, :] * sb.astype(np.float32)[None, :, :]).astype(np.float64)
    # s: [M, NB, KB] -> per (m, n, kb)
    nb_of_n = np.arange(N) // 128
    out = np.zeros((M, N))
    for kb in range(K // 128):
        P = A[:, kb * 128:(kb + 1) * 128] @ B[:, kb * 128:(kb + 1) * 128].T
        out += s[:, nb_of_n, kb] * P
    return out


def test_decoder_matches_torch_on_every_code():
    b = np.arange(256, dtype=np.uint8)
    got = oracle.e4m3fn_to_f64(b)
    want = torch.from_numpy(b).view(FP8).to(torch.float64).numpy()
    assert np.array_equal(got, want, equal_nan=True)
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and np.isnan(got[0x7F])


@pytest.mark.parametrize("M,N,K", [(5, 128, 128), (33, 272, 384), (64, 384, 1024), (7, 2112, 256)])
@pytest.mark.parametrize("afmt,bfmt,layout", [("f32", "f32", oracle.L_COL),
                                              ("f32", "f32", oracle.L_ROW),
                                              ("ue8m0", "ue8m0", oracle.L_COL),
                                              ("ue8m0", "f32", oracle.L_COL),
                                              ("f32", "ue8m0", oracle.L_ROW)])
def test_oracle_matches_dequantized_matmul(M, N, K, afmt, bfmt, layout):
    rng = np.random.default_rng(M * 131 + N + K)
    kb, nb = K // 128, (N + 127) // 128
    a_q, b_q = rand_fp8(rng, (M, K)), rand_fp8(rng, (N, K))
    a_s = rand_scales(rng, (kb, M) if layout == oracle.L_COL else (M, kb), afmt)
    b_s = rand_scales(rng, (nb, kb), bfmt)
    c, bound = oracle.gemm(a_q, a_s, b_q, b_s, a_layout=layout)
    ref = dequant_ref(a_q, a_s, b_q, b_s, layout)
    # The two differ only by double rounding of the scaled block sums.
    assert np.all(np.abs(c - ref) <= 1e-12 * bound + 1e-300)
    assert np.all(np.abs(c) <= bound * (1 + 1e-12))


def test_one_hot_rows_select_scaled_weights():
    M, N, K = 4, 256, 256
    rng = np.random.default_rng(7)
    b_q = rand_fp8(rng, (N, K))
    a = np.zeros((M, K), np.float32)
    cols = [3, 130, 255, 0]
    for m, k in enumerate(cols):
        a[m, k] = 1.0
    a_q = torch.from_numpy(a).to(FP8).view(torch.uint8).numpy()
    a_s = np.full((K // 128, M), 0.5, np.float32)                 # column-major
    b_s = np.array([[2.0, 4.0], [8.0, 16.0]], np.float32)         # [N/128, K/128]
    c, _ = oracle.gemm(a_q, a_s, b_q, b_s)
    B = oracle.e4m3fn_to_f64(b_q)
    for m, k in enumerate(cols):
        kb = k // 128
        want = 0.5 * b_s[np.arange(N) // 128, kb] * B[:, k]
        assert np.array_equal(c[m], want)


def test_power_of_two_scales_are_exact():
    # UE8M0 scales: C is an exact dyadic sum; compare with exact integer math.
    M, N, K = 3, 128, 256
    rng = np.random.default_rng(3)
    ints = rng.integers(-8, 9, size=(M, K)).astype(np.float32)
    intsb = rng.integers(-8, 9, size=(N, K)).astype(np.float32)
    a_q = torch.from_numpy(ints).to(FP8).view(torch.uint8).numpy()
    b_q = torch.from_numpy(intsb).to(FP8).view(torch.uint8).numpy()
    a_s = np.array([[127, 128, 126], [130, 127, 120]], np.uint8)   # [K/128, M]
    b_s = np.array([[127, 125]], np.uint8)
    c, _ = oracle.gemm(a_q, a_s, b_q, b_s)
    want = np.zeros((M, N))
    for kb in range(2):
        P = ints[:, kb * 128:(kb + 1) * 128].astype(np.int64) @ \
            intsb[:, kb * 128:(kb + 1) * 128].astype(np.int64).T
        want += P * np.ldexp(1.0, a_s[kb].astype(np.int64) - 127)[:, None] * \
            np.ldexp(1.0, int(b_s[0, kb]) - 127)
    assert np.array_equal(c, want)
