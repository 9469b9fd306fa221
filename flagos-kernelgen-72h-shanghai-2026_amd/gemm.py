"""fp8 block-scaled GEMM that consumes the quantizer's output.

``fp8_block_scaled_gemm(a_q, a_scale, b_q, b_scale)`` computes

    C[m, n] = sum_kb  sa[m, kb] * sb[n // 128, kb] * sum_{k in kb} A[m, k] * B[n, k]

in bf16, i.e. ``(A * sa) @ (B * sb).T`` with 1 x 128 activation scales and
128 x 128 weight-block scales: the DeepSeek-V3 style fp8 linear layer whose
input format (fp8 codes plus column-major fp32 or UE8M0 scales) is what
``fused_add_rmsnorm_group_quant`` writes.  The kernel is libfagq.so's
``fagq_gemm_launch`` (include/fagq_gemm.h); there is no fallback.

No counterpart in the reference repository: its operator
(src/task01_fused_add_rmsnorm_group_quant.py:1731-1851) stops at the
quantized tensor and scales.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_FP8 = torch.float8_e4m3fn
BLOCK = 128


def _scale_format(t: torch.Tensor, what: str) -> int:
    if t.dtype == torch.float32:
        return _lib.SCALE_F32
    if t.dtype == torch.uint8:
        return _lib.SCALE_UE8M0
    raise TypeError(f"{what} must be float32 or uint8 (ue8m0), got {t.dtype}")


def fp8_block_scaled_gemm(a_q: torch.Tensor, a_scale: torch.Tensor, b_q: torch.Tensor,
                          b_scale: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """a_q: float8_e4m3fn [M, K]; a_scale: float32 / uint8 [M, K/128], row-major or
    column-major (strides (1, M), as the quantizer writes it); b_q: float8_e4m3fn
    [N, K]; b_scale: float32 / uint8 [ceil(N/128), K/128] contiguous.  Returns
    (or fills) a bf16 [M, N] tensor, asynchronously on the current stream."""
    if a_q.dtype != _FP8 or b_q.dtype != _FP8:
        raise TypeError("a_q and b_q must be float8_e4m3fn")
    if a_q.dim() != 2 or b_q.dim() != 2 or a_q.shape[1] != b_q.shape[1]:
        raise ValueError(f"a_q [M, K] and b_q [N, K] must share K: {tuple(a_q.shape)}, "
                         f"{tuple(b_q.shape)}")
    M, K = a_q.shape
    N = b_q.shape[0]
    if K % BLOCK or N % 16:
        raise ValueError(f"K must be a multiple of {BLOCK} and N of 16 (K={K}, N={N})")
    if not (a_q.is_contiguous() and b_q.is_contiguous()):
        raise ValueError("a_q and b_q must be contiguous")
    kb = K // BLOCK
    asf = _scale_format(a_scale, "a_scale")
    bsf = _scale_format(b_scale, "b_scale")
    if tuple(a_scale.shape) != (M, kb):
        raise ValueError(f"a_scale must have shape ({M}, {kb}), got {tuple(a_scale.shape)}")
    if a_scale.is_contiguous():
        layout = _lib.LAYOUT_ROW_MAJOR
    elif a_scale.stride() == (1, M):
        layout = _lib.LAYOUT_COL_MAJOR
    else:
        raise ValueError(f"a_scale must be row-major or column-major, strides {a_scale.stride()}")
    nb = (N + BLOCK - 1) // BLOCK
    if tuple(b_scale.shape) != (nb, kb) or not b_scale.is_contiguous():
        raise ValueError(f"b_scale must be a contiguous ({nb}, {kb}) tensor")
    dev = a_q.device
    if dev.type != "cuda" or any(t.device != dev for t in (a_scale, b_q, b_scale)):
        raise ValueError("all tensors must be on the same GPU")
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or not out.is_contiguous() \
            or out.device != dev:
        raise ValueError(f"out must be a contiguous bf16 [{M}, {N}] tensor on {dev}")
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        st = lib.fagq_gemm_launch(P(a_q), P(a_scale), P(b_q), P(b_scale), P(out), M, N, K, asf,
                                  layout, bsf, ctypes.c_void_p(stream))
    _lib.check(st, "fagq_gemm_launch")
    return out


def gemm_route(M: int, N: int, K: int) -> dict:
    r = _lib.GemmRoute()
    _lib.check(_lib.load().fagq_gemm_query_route(M, N, K, ctypes.byref(r)), "fagq_gemm_query_route")
    return {f: getattr(r, f) for f, _ in _lib.GemmRoute._fields_}
