"""MLA backward, NoPE, shared K = V = C (Task 03 of the reference repository).

``mla_bwd_nope_dkdv`` keeps the reference's signature and destination-passing
semantics (src/task03_mla_bwd_nope_dkdv.py:453-480) and computes what the
reference's GPU path computes (_run_gpu, :401-425): the exact gradient for
the first min(16, S) query rows of every head, ``dq = sm_scale * do`` for the
other rows, and ``dc_kv[b, j] = sum_{i >= j} sum_h do[b, h, i] / (i + 1)``,
the uniform-causal approximation of reports/task03_mla_bwd_nope_dkdv.md:160-176.
That is not the exact attention backward for general inputs; it is the
reference's operator.  The kernels are libfagq.so's ``fagq_mla_bwd_launch``
(include/fagq_mla.h); there is no fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

MLA_F32, MLA_BF16 = 0, 1
EXACT_ROWS = 16
SLICE_D = 512     # dims per column slice of the kernels (include/fagq_mla.h)


def _out_code(t: torch.Tensor, name: str) -> int:
    if t.dtype == torch.float32:
        return MLA_F32
    if t.dtype == torch.bfloat16:
        return MLA_BF16
    raise TypeError(f"{name} must be float32 or bfloat16, got {t.dtype}")


def workspace_bytes(B: int, S: int, D: int) -> int:
    n = _lib.load().fagq_mla_bwd_workspace_bytes(B, S, D)
    if n < 0:
        raise ValueError(f"no workspace size for B={B}, S={S}, D={D}")
    return n


def check_workspace(workspace: torch.Tensor, need: int, dev: torch.device) -> None:
    """A caller's workspace must be a contiguous tensor on ``dev`` whose own bytes
    and whose storage past its offset both hold ``need`` bytes: the kernels write
    ``need`` contiguous bytes from ``data_ptr()``, so a strided or expanded view
    would let them write outside the view or its storage."""
    if workspace.device != dev or not workspace.is_contiguous():
        raise ValueError(f"workspace must be a contiguous tensor on {dev}")
    nbytes = workspace.numel() * workspace.element_size()
    room = (workspace.untyped_storage().nbytes()
            - workspace.storage_offset() * workspace.element_size())
    if min(nbytes, room) < need:
        raise ValueError(f"workspace must hold {need} bytes on {dev}, got {min(nbytes, room)}")


def mla_bwd_nope_dkdv(q: torch.Tensor, c_kv: torch.Tensor, out: torch.Tensor, do: torch.Tensor,
                      lse: torch.Tensor, dq: torch.Tensor, dc_kv: torch.Tensor, sm_scale: float,
                      workspace: torch.Tensor | None = None):
    """q, out, do: bfloat16 [B, H, S, D]; c_kv: bfloat16 [B, S, D]; lse: float32
    [B, H, S]; dq [B, H, S, D] and dc_kv [B, S, D]: float32 or bfloat16.  All
    contiguous, on one GPU.  ``workspace`` (optional): a uint8 GPU tensor of at
    least ``workspace_bytes(B, S, D)`` bytes; allocated per call when absent,
    as the reference allocates its head-sum buffer.  Returns ``(dq, dc_kv)``."""
    if q.dim() != 4:
        raise ValueError(f"q must be [B, H, S, D], got shape {tuple(q.shape)}")
    B, H, S, D = (int(s) for s in q.shape)
    dev = q.device
    if dev.type != "cuda":
        raise ValueError("q must be a GPU (HIP) tensor; this operator has no CPU path")
    for name, t, shape, dts in (("q", q, (B, H, S, D), (torch.bfloat16,)),
                                ("c_kv", c_kv, (B, S, D), (torch.bfloat16,)),
                                ("out", out, (B, H, S, D), (torch.bfloat16,)),
                                ("do", do, (B, H, S, D), (torch.bfloat16,)),
                                ("lse", lse, (B, H, S), (torch.float32,)),
                                ("dq", dq, (B, H, S, D), (torch.float32, torch.bfloat16)),
                                ("dc_kv", dc_kv, (B, S, D), (torch.float32, torch.bfloat16))):
        if t.device != dev or t.dtype not in dts or tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {'/'.join(map(str, dts))} tensor of "
                             f"shape {shape} on {dev}")
    need = workspace_bytes(B, S, D)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    else:
        check_workspace(workspace, need, dev)
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        st = lib.fagq_mla_bwd_launch(P(q), P(c_kv), P(out), P(do), P(lse), P(dq), P(dc_kv),
                                     P(workspace), workspace.numel() * workspace.element_size(),
                                     B, H, S, D, float(sm_scale), _out_code(dq, "dq"),
                                     _out_code(dc_kv, "dc_kv"), ctypes.c_void_p(stream))
    _lib.check(st, "fagq_mla_bwd_launch")
    return dq, dc_kv
