"""DSA top-k page-table transform (Task 02 of the reference repository).

``dsa_topk_page_table_transform`` keeps the reference's signature and
destination-passing semantics (src/task02_dsa_topk_page_table_transform.py:1666,
returns at :1726): for every query row of ``scores[B, H, Q, NB]`` the blocks
of the causal valid prefix (from ``q_pos``, ``kv_lens`` and ``block_size``)
are ordered by score descending, then block id ascending; the first
``top_k`` ids go to ``out_blocks`` and their ``page_table[b, id]`` entries to
``out_pages`` (-1 past the number of selectable blocks).  The kernel is
libfagq.so's ``fagq_dsa_topk_launch`` (include/fagq_dsa.h); there is no
fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

DSA_F32, DSA_BF16 = 0, 1
DSA_I32, DSA_I64 = 0, 1
MAX_NB, MAX_TOP_K = 1 << 28, 1024


def dsa_topk_page_table_transform(scores: torch.Tensor, page_table: torch.Tensor,
                                  q_pos: torch.Tensor, kv_lens: torch.Tensor,
                                  out_blocks: torch.Tensor, out_pages: torch.Tensor,
                                  block_size: int, top_k: int):
    """scores: float32 or bfloat16 [B, H, Q, NB] contiguous; page_table: int32 [B, NB];
    q_pos: [B, Q] and kv_lens: [B], both int32 or both int64; out_blocks, out_pages:
    int32 [B, H, Q, top_k].  Returns ``(out_blocks, out_pages)``."""
    if scores.dim() != 4:
        raise ValueError(f"scores must be [B, H, Q, NB], got shape {tuple(scores.shape)}")
    B, H, Q, NB = (int(s) for s in scores.shape)
    top_k, block_size = int(top_k), int(block_size)
    if scores.dtype == torch.float32:
        sdt = DSA_F32
    elif scores.dtype == torch.bfloat16:
        sdt = DSA_BF16
    else:
        raise TypeError(f"scores must be float32 or bfloat16, got {scores.dtype}")
    if q_pos.dtype != kv_lens.dtype or q_pos.dtype not in (torch.int32, torch.int64):
        raise TypeError("q_pos and kv_lens must both be int32 or both int64")
    idt = DSA_I64 if q_pos.dtype == torch.int64 else DSA_I32
    dev = scores.device
    if dev.type != "cuda":
        raise ValueError("scores must be a GPU (HIP) tensor; this operator has no CPU path")
    for name, t, shape, dt in (("page_table", page_table, (B, NB), torch.int32),
                               ("q_pos", q_pos, (B, Q), q_pos.dtype),
                               ("kv_lens", kv_lens, (B,), q_pos.dtype),
                               ("out_blocks", out_blocks, (B, H, Q, top_k), torch.int32),
                               ("out_pages", out_pages, (B, H, Q, top_k), torch.int32)):
        if t.device != dev or t.dtype != dt or tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dt} tensor of shape {shape} on {dev}")
    if not scores.is_contiguous():
        raise ValueError("scores must be contiguous")
    lib = _lib.load()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        st = lib.fagq_dsa_topk_launch(P(scores), sdt, P(page_table), P(q_pos), P(kv_lens), idt,
                                      P(out_blocks), P(out_pages), B, H, Q, NB, block_size, top_k,
                                      ctypes.c_void_p(stream))
    _lib.check(st, "fagq_dsa_topk_launch")
    return out_blocks, out_pages
