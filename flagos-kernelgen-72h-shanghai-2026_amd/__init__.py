"""MI355X (gfx950) fused residual-add + RMSNorm + per-token-group quantization.

Drop-in for the Task 01 operator of sinpeyw/flagos-kernelgen-72h-shanghai-2026
(src/task01_fused_add_rmsnorm_group_quant.py:1731), backed by hand-written HIP
kernels in libfagq.so (C ABI: include/fagq.h).  The directory name is not a
Python identifier; load it with ``__graft_entry__.load_package()``, which
registers it as ``fagq_mi355x``.
"""
from . import _lib
from ._lib import FagqError, load as load_library, load_probe as load_probe_library
from .dsa_topk import dsa_topk_page_table_transform
from .gemm import fp8_block_scaled_gemm, gemm_route
from .mla_bwd import mla_bwd_nope_dkdv
from .ops import (empty_scales, fused_add_rmsnorm_group_quant, fused_add_rmsnorm_group_quant_fn,
                  fused_reduce_add_rmsnorm_group_quant, route_for)

__all__ = [
    "FagqError",
    "dsa_topk_page_table_transform",
    "empty_scales",
    "fp8_block_scaled_gemm",
    "fused_add_rmsnorm_group_quant",
    "fused_add_rmsnorm_group_quant_fn",
    "fused_reduce_add_rmsnorm_group_quant",
    "gemm_route",
    "load_library",
    "load_probe_library",
    "mla_bwd_nope_dkdv",
    "route_for",
]
