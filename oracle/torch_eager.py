"""Eager-PyTorch CPU restatement of the operator (TEST INFRASTRUCTURE ONLY).

The reference repository ships no CPU or PyTorch path; its math lives in
Triton kernels (src/task01_fused_add_rmsnorm_group_quant.py:65-121 and
:1066-1348).  This module restates the same formulas with PyTorch CPU ops,
in the same operation order as the C oracle, so that bench.py can time "the
reference's CPU PyTorch path" on the host cores.  tests/ check it
bit-for-bit against the C oracle.
"""
from __future__ import annotations

import torch


def fagq_torch(x: torch.Tensor, residual: torch.Tensor, gamma: torch.Tensor, eps: float,
               group_size: int, out_dtype: torch.dtype = torch.float8_e4m3fn,
               scale_ue8m0: bool = False, col_major: bool = False, rounding: str = "rne",
               with_norm: bool = False):
    """x, residual: [M, D]; gamma: [D] (CPU tensors; bf16, or the typed form's
    element types: x and gamma one type, residual another).

    Returns (residual_out in residual's type, q, scale[, norm_out in x's type])
    with scale in its physical layout ([M, groups] or [groups, M]).
    """
    M, D = x.shape
    G = group_size
    groups = D // G
    qmax = 448.0 if out_dtype == torch.float8_e4m3fn else 127.0
    r = x.float() + residual.float()                                # :88-89
    residual_out = r.to(residual.dtype)                             # :91
    rd = r.double()
    sumsq = (rd * rd).sum(dim=1).float()                            # :90, exact-rounded
    mean = sumsq / torch.tensor(float(D), dtype=torch.float32)
    v = mean + torch.tensor(eps, dtype=torch.float32)
    inv = (1.0 / torch.sqrt(v.double())).float()                    # :100
    w = r * gamma.float()                                           # :93-94
    gmax = w.abs().view(M, groups, G).amax(dim=2)                   # :95-98
    inv_q = inv / torch.tensor(qmax, dtype=torch.float32)
    s = torch.clamp_min(gmax * inv_q[:, None], torch.tensor(1e-12, dtype=torch.float32))  # :102
    n = w * inv[:, None]                                            # :101
    if scale_ue8m0:
        bits = s.view(torch.int32)
        e = (bits >> 23) - 127 + ((bits & 0x7FFFFF) != 0).to(torch.int32)
        e = torch.clamp_max(e, 127)
        mult = torch.pow(torch.tensor(2.0, dtype=torch.float64), (-e).double()).float()
        u = n.view(M, groups, G) * mult[..., None]
        scale = (e + 127).to(torch.uint8)
    else:
        mul = torch.ones_like(s) / s                                # :103
        u = n.view(M, groups, G) * mul[..., None]
        scale = s
    t = torch.clamp(u, -qmax, qmax).view(M, D)                      # :112-116
    if out_dtype == torch.float8_e4m3fn:
        q = t.to(torch.float8_e4m3fn)
    elif rounding == "rne":
        q = torch.round(t).to(torch.int8)
    else:
        q = t.to(torch.int8)                                        # truncation, as fp_to_si
    if col_major:
        scale = scale.t().contiguous()
    outs = (residual_out, q, scale)
    if with_norm:
        outs = outs + (n.to(x.dtype),)
    return outs
