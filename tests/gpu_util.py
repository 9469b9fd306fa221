"""Helpers shared by the GPU parity tests: run the HIP library and the CPU
oracle on the same bf16 inputs and return numpy views of both."""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import torch

import oracle

FMTS = {   # name -> (torch dtype, rounding, oracle q_format, oracle rounding)
    "fp8": (torch.float8_e4m3fn, "rne", oracle.Q_FP8, oracle.R_RNE),
    "int8_rne": (torch.int8, "rne", oracle.Q_INT8, oracle.R_RNE),
    "int8_trunc": (torch.int8, "trunc", oracle.Q_INT8, oracle.R_TRUNC),
}


def note(msg: str) -> None:
    """Names the case on stdout before each GPU step."""
    print(msg, flush=True)
    sys.stdout.flush()


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint16).numpy()


def run_ref(x, r, g, G, fmt, ue8m0=False, col=False, eps=1e-6, with_norm=False):
    _, _, qf, rnd = FMTS[fmt]
    return oracle.fagq(u16(x), u16(r), u16(g), eps, G, qf,
                       oracle.S_UE8M0 if ue8m0 else oracle.S_F32,
                       oracle.L_COL if col else oracle.L_ROW, rnd, with_norm)


def to_numpy(ro, q, sc, norm, col):
    phys = sc.t() if col else sc
    out = {"residual_out": ro.cpu().view(torch.uint16).numpy(),
           "q": q.cpu().view(torch.uint8).numpy(),
           "scale": np.ascontiguousarray(phys.cpu().numpy())}
    if norm is not None:
        out["norm_out"] = norm.cpu().view(torch.uint16).numpy()
    return out


def run_gpu(pkg, dev, x, r, g, G, fmt, ue8m0=False, col=False, eps=1e-6, with_norm=False,
            mapping=None, inplace=False, stream=None, scale_offset=0):
    """Runs the library on cuda tensors copied from the CPU inputs.
    mapping = (waves_per_row, rows_per_block, row_group_mode, xcd_remap[, lds_bytes]) forces a
    launch mapping through fagq_launch_mapped; otherwise the public Python operator
    (reference signature) is used.  scale_offset > 0 places the scales that many
    elements past an aligned allocation (a misaligned scale pointer)."""
    qdt, rnd, _, _ = FMTS[fmt]
    M, D = x.shape
    xd, rd, gd = x.to(dev), r.to(dev), g.to(dev)
    ro = rd if inplace else torch.empty_like(rd)
    q = torch.empty((M, D), dtype=qdt, device=dev)
    if scale_offset:
        dt = torch.uint8 if ue8m0 else torch.float32
        buf = torch.empty(M * (D // G) + scale_offset, dtype=dt, device=dev)[scale_offset:]
        sc = buf.view(D // G, M).t() if col else buf.view(M, D // G)
    else:
        sc = pkg.empty_scales(M, D // G, ue8m0=ue8m0, col_major=col, device=dev)
    norm = torch.empty_like(xd) if with_norm else None
    if mapping is None:
        ctx = torch.cuda.stream(stream) if stream is not None else torch.cuda.stream(torch.cuda.current_stream(dev))
        with ctx:
            pkg.fused_add_rmsnorm_group_quant(xd, rd, gd, ro, norm, q, sc, eps, G,
                                              rounding=rnd if qdt == torch.int8 else None)
    else:
        from fagq_mi355x import _lib
        wpr, rpb, mode, remap, *rest = mapping
        lds = rest[0] if rest else 0
        p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
        st = pkg.load_library().fagq_launch_mapped(
            p(xd), p(rd), p(gd), p(ro), p(norm), p(q), p(sc), M, D, G, eps,
            _lib.Q_FP8_E4M3FN if qdt == torch.float8_e4m3fn else _lib.Q_INT8,
            _lib.SCALE_UE8M0 if ue8m0 else _lib.SCALE_F32,
            _lib.LAYOUT_COL_MAJOR if col else _lib.LAYOUT_ROW_MAJOR,
            _lib.ROUND_RNE if rnd == "rne" else _lib.ROUND_TRUNC, wpr, rpb, mode, remap, lds,
            ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
        _lib.check(st, "fagq_launch_mapped")
    torch.cuda.synchronize(dev)
    return to_numpy(ro, q, sc, norm, col)
