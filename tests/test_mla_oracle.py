"""Pins the CPU oracle of the Task 03 operator (oracle/mla_bwd_oracle.c), the
function the reference's GPU path computes (src/task03_mla_bwd_nope_dkdv.py:401-425).

The reference holds no tests or vectors for Task 03.  The oracle is pinned by
the mathematics of attention backward with shared K = V = C, computed
independently by torch autograd in float64:
* the first min(16, S) rows of dq are the exact gradient, up to the bf16
  rounding of P and dS the reference applies;
* with q = 0 the attention is exactly uniform over the causal window and the
  dK part of dC vanishes, so the reference's uniform-causal dC formula is the
  exact gradient there;
* rows >= 16 of dq are fp32(do) * sm_scale (reports/task03_...md:146-152);
* the reverse scan equals a numpy restatement of dc_j = sum_{i >= j} hs_i / (i + 1).
"""
import numpy as np
import pytest
import torch

import oracle

F64 = torch.float64


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.uint16).numpy()


def bf16_vals(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float64)


def forward(q, c, scale, with_p=False):
    """Causal attention with K = V = C: q [B, H, S, D], c [B, S, D] (float64)."""
    S = q.shape[2]
    logits = torch.einsum("bhsd,btd->bhst", q, c) * scale
    mask = torch.ones(S, S, dtype=torch.bool).tril()
    logits = logits.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(logits, -1)
    p = torch.softmax(logits, -1)
    out = torch.einsum("bhst,btd->bhsd", p, c)
    return (out, lse, p) if with_p else (out, lse)


def exact_grads(q, c, do, scale):
    q = q.clone().requires_grad_(True)
    c = c.clone().requires_grad_(True)
    out, _ = forward(q, c, scale)
    out.backward(do)
    return q.grad, c.grad


def make_case(seed, B=1, H=3, S=40, D=64, qscale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = bf16_vals(torch.randn(B, H, S, D, generator=g, dtype=F64) * qscale)
    c = bf16_vals(torch.randn(B, S, D, generator=g, dtype=F64))
    do = bf16_vals(torch.randn(B, H, S, D, generator=g, dtype=F64))
    scale = D ** -0.5
    out, lse = forward(q, c, scale)
    return q, c, bf16_vals(out), do, lse.float(), scale


def run_oracle(q, c, out, do, lse, scale):
    return oracle.mla_bwd(bf16_bits(q), bf16_bits(c), bf16_bits(out), bf16_bits(do),
                          lse.numpy(), scale)


@pytest.mark.parametrize("seed,S,D", [(0, 40, 64), (1, 16, 128), (2, 100, 64), (3, 7, 64)])
def test_exact_rows_match_autograd(seed, S, D):
    q, c, out, do, lse, scale = make_case(seed, S=S, D=D)
    dq, _, bound = run_oracle(q, c, out, do, lse, scale)
    bound = bound[0]
    dq_ex, _ = exact_grads(q, c, do, scale)
    # out enters as bf16: delta_i = out_i . do_i moves by ddelta_i, which moves
    # the exact dq_i by -scale ddelta_i (P c)_i.  Apply that, then only the
    # bf16 rounding of P and dS (2^-9 relative each) remains.
    out_ex, _, p = forward(q, c, scale, with_p=True)
    ddelta = ((out - out_ex) * do).sum(-1)
    want = dq_ex - scale * ddelta[..., None] * torch.einsum("bhst,btd->bhsd", p, c)
    E = min(16, S)
    err = np.abs(dq[:, :, :E] - want[:, :, :E].numpy())
    tol = 2.0 ** -7 * bound + 1e-12
    assert (err <= tol).all(), float((err - tol).max())
    # the tolerance is tight enough to see a plausible mistake: a dropped sm_scale in dS
    assert np.abs(want[:, :, :E].numpy() / scale - dq[:, :, :E]).max() > tol.max()


@pytest.mark.parametrize("seed,B,H,S", [(4, 1, 4, 50), (5, 2, 2, 33)])
def test_dc_is_the_exact_gradient_for_uniform_attention(seed, B, H, S):
    q, c, out, do, lse, scale = make_case(seed, B=B, H=H, S=S, qscale=0.0)
    _, dc, _ = run_oracle(q, c, out, do, lse, scale)
    _, dc_ex = exact_grads(q, c, do, scale)
    np.testing.assert_allclose(dc, dc_ex.numpy(), rtol=1e-10, atol=1e-12)


def test_dc_differs_from_the_exact_gradient_in_general():
    # With non-zero q the reference's dC is an approximation (its report says so).
    q, c, out, do, lse, scale = make_case(6, S=48, qscale=1.0)
    _, dc, _ = run_oracle(q, c, out, do, lse, scale)
    _, dc_ex = exact_grads(q, c, do, scale)
    assert np.abs(dc - dc_ex.numpy()).max() > 1e-3


def test_rows_past_the_prefix_are_scaled_do_and_scan_matches_numpy():
    q, c, out, do, lse, scale = make_case(7, B=2, H=3, S=70, D=64)
    dq, dc, _ = run_oracle(q, c, out, do, lse, scale)
    do32 = do.float().numpy()
    want = (do32 * np.float32(scale)).astype(np.float32)
    assert np.array_equal(dq[:, :, 16:], want[:, :, 16:].astype(np.float64))
    hs = do.numpy().sum(1) / np.arange(1, 71)[None, :, None]
    want_dc = np.flip(np.cumsum(np.flip(hs, 1), 1), 1)
    np.testing.assert_allclose(dc, want_dc, rtol=1e-12, atol=1e-12)


def test_round_bf16_is_round_to_nearest_even():
    # P and dS are rounded like torch's fp32 -> bf16 cast: pinned through the
    # exact rows, where a single dS entry (one key) makes dq = dS * c exact.
    q, c, out, do, lse, scale = make_case(8, S=1, D=64)
    dq, _, _ = run_oracle(q, c, out, do, lse, scale)
    p = torch.exp((q[0, :, 0] @ c[0, 0]) * scale - lse[0, :, 0].double()).float().to(torch.bfloat16)
    dp = do[0, :, 0] @ c[0, 0]
    delta = (out[0, :, 0] * do[0, :, 0]).sum(-1)
    ds = (p.float().double() * (dp - delta) * scale).float().to(torch.bfloat16).double()
    want = ds[:, None] * c[0, 0][None, :]
    np.testing.assert_allclose(dq[0, :, 0], want.numpy(), rtol=1e-12, atol=1e-12)
