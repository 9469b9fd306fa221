"""CPU oracle for the fused residual-add + RMSNorm + group-quant operator.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this package, and only as the checker
(or, for the baseline, as the CPU path being timed); the product library
never loads it.

Two restatements of the reference algorithm
(sinpeyw/flagos-kernelgen-72h-shanghai-2026,
src/task01_fused_add_rmsnorm_group_quant.py:65-121 and :1066-1348):

* ``fagq`` - the C restatement in fagq_oracle.c (scalar, OpenMP over rows),
  called through ctypes on numpy arrays.  This is the parity reference.
* ``torch_eager.fagq_torch`` - the same formulas as eager PyTorch CPU ops,
  the "CPU PyTorch path" that the benchmark times as its CPU baseline.
* ``gemm`` - gemm_oracle.c, the fp8 block-scaled GEMM that consumes the
  operator's codes and scales (no reference counterpart; its definition is
  in include/fagq_gemm.h).
* ``dsa_topk`` - dsa_topk_oracle.c, the Task 02 DSA top-k page-table
  transform (src/task02_dsa_topk_page_table_transform.py:154-175).

bf16 tensors are passed as their uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
# FAGQ_TEST_ORACLE_LIBRARY: the tests' sanitizer run loads a sanitizer build of
# the same sources instead.
LIB_PATH = Path(os.environ.get("FAGQ_TEST_ORACLE_LIBRARY") or ORACLE_DIR / "libfagq_oracle.so")

Q_INT8, Q_FP8 = 0, 1
S_F32, S_UE8M0 = 0, 1
L_ROW, L_COL = 0, 1
R_RNE, R_TRUNC = 0, 1

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from . import build as _build
            _build.build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I64, I, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.orc_bf16_from_f32.argtypes = [P, P, I64]
        L.orc_bf16_from_f32.restype = None
        L.orc_encode.argtypes = [P, P, I64, I, I]
        L.orc_encode.restype = None
        L.orc_e4m3fn_raw.argtypes = [P, P, I64]
        L.orc_e4m3fn_raw.restype = None
        L.orc_ceil_log2.argtypes = [P, P, I64]
        L.orc_ceil_log2.restype = None
        L.orc_fagq.argtypes = [P, P, P, P, P, P, P, I64, I64, I64, F, I, I, I, I, I]
        L.orc_fagq.restype = I
        L.orc_fagq_parts.argtypes = [P, I] + [P] * 6 + [I64, I64, I64, F, I, I, I, I, I]
        L.orc_fagq_parts.restype = I
        L.orc_fagq_typed.argtypes = [P] * 7 + [I64, I64, I64, F, I, I, I, I, I, I, I]
        L.orc_fagq_typed.restype = I
        L.orc_f16_from_f32.argtypes = [P, P, I64]
        L.orc_f16_from_f32.restype = None
        L.orc_f32_from_f16.argtypes = [P, P, I64]
        L.orc_f32_from_f16.restype = None
        L.orc_e4m3fn_to_f64.argtypes = [P, P, I64]
        L.orc_e4m3fn_to_f64.restype = None
        L.orc_gemm.argtypes = [P, P, P, P, P, P, I64, I64, I64, I, I, I, I]
        L.orc_gemm.restype = I
        L.orc_dsa_topk.argtypes = [P, I, P, P, P, I, P, P, I64, I64, I64, I64, I64, I64, I]
        L.orc_mla_bwd.restype = I
        L.orc_mla_bwd.argtypes = [P] * 8 + [I64] * 4 + [F, I]
        L.orc_dsa_topk.restype = I
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def bf16_from_f32(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, np.uint16)
    lib().orc_bf16_from_f32(_ptr(v), _ptr(out), v.size)
    return out


def f16_from_f32(v: np.ndarray) -> np.ndarray:
    """fp32 -> IEEE binary16 bits, round to nearest even (the oracle's encoder)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, np.uint16)
    lib().orc_f16_from_f32(_ptr(v), _ptr(out), v.size)
    return out


def f32_from_f16(h: np.ndarray) -> np.ndarray:
    """IEEE binary16 bits -> fp32 (the oracle's decoder)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f32_from_f16(_ptr(h), _ptr(out), h.size)
    return out


def f32_from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def encode(t: np.ndarray, q_format: int, rounding: int = R_RNE) -> np.ndarray:
    """Codes for already-scaled values, after the operator's clamp to +-QMAX."""
    t = np.ascontiguousarray(t, dtype=np.float32)
    out = np.empty(t.shape, np.uint8)
    lib().orc_encode(_ptr(t), _ptr(out), t.size, q_format, rounding)
    return out


def e4m3fn_raw(v: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn bits, round-to-nearest-even, no clamp (overflow -> NaN)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, np.uint8)
    lib().orc_e4m3fn_raw(_ptr(v), _ptr(out), v.size)
    return out


def ceil_log2(s: np.ndarray) -> np.ndarray:
    s = np.ascontiguousarray(s, dtype=np.float32)
    out = np.empty(s.shape, np.int32)
    lib().orc_ceil_log2(_ptr(s), _ptr(out), s.size)
    return out


def fagq(x: np.ndarray, residual: np.ndarray, gamma: np.ndarray, eps: float, group_size: int,
         q_format: int = Q_FP8, scale_format: int = S_F32, scale_layout: int = L_ROW,
         rounding: int = R_RNE, with_norm: bool = False, nthreads: int = 0) -> dict:
    """Runs the C restatement.  x, residual: uint16 [M, D] (bf16 bits);
    gamma: uint16 [D].  Returns residual_out (uint16), q (uint8 codes),
    scale (float32 or uint8, physical layout [M, groups] or [groups, M]) and
    norm_out (uint16) when with_norm."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    residual = np.ascontiguousarray(residual, dtype=np.uint16)
    gamma = np.ascontiguousarray(gamma, dtype=np.uint16)
    M, D = x.shape
    assert residual.shape == (M, D) and gamma.shape == (D,)
    groups = D // group_size
    res_out = np.empty((M, D), np.uint16)
    norm_out = np.empty((M, D), np.uint16) if with_norm else None
    q = np.empty((M, D), np.uint8)
    sdt = np.float32 if scale_format == S_F32 else np.uint8
    scale = np.empty((groups, M) if scale_layout == L_COL else (M, groups), sdt)
    st = lib().orc_fagq(_ptr(x), _ptr(residual), _ptr(gamma), _ptr(res_out), _ptr(norm_out),
                        _ptr(q), _ptr(scale), M, D, group_size, float(eps), q_format,
                        scale_format, scale_layout, rounding, nthreads)
    if st != 0:
        raise ValueError(f"oracle rejected the arguments (status {st})")
    out = {"residual_out": res_out, "q": q, "scale": scale}
    if with_norm:
        out["norm_out"] = norm_out
    return out


DT_BF16, DT_F16, DT_F32 = 0, 1, 2
_DT_NP = {DT_BF16: np.uint16, DT_F16: np.uint16, DT_F32: np.float32}


def fagq_typed(x: np.ndarray, residual: np.ndarray, gamma: np.ndarray, eps: float,
               group_size: int, act_dtype: int, res_dtype: int, q_format: int = Q_FP8,
               scale_format: int = S_F32, scale_layout: int = L_ROW, rounding: int = R_RNE,
               with_norm: bool = False, nthreads: int = 0) -> dict:
    """The typed form (orc_fagq_typed): x and gamma hold act_dtype elements,
    residual res_dtype elements (bf16 and fp16 as uint16 bit patterns, fp32 as
    float32).  Returns residual_out (res_dtype storage), q, scale and, when
    with_norm, norm_out (act_dtype storage)."""
    ta, tr = _DT_NP[act_dtype], _DT_NP[res_dtype]
    x = np.ascontiguousarray(x).view(ta) if x.dtype.itemsize == np.dtype(ta).itemsize else None
    residual = np.ascontiguousarray(residual).view(tr)
    gamma = np.ascontiguousarray(gamma).view(ta)
    assert x is not None
    M, D = x.shape
    assert residual.shape == (M, D) and gamma.shape == (D,)
    groups = D // group_size
    res_out = np.empty((M, D), tr)
    norm_out = np.empty((M, D), ta) if with_norm else None
    q = np.empty((M, D), np.uint8)
    sdt = np.float32 if scale_format == S_F32 else np.uint8
    scale = np.empty((groups, M) if scale_layout == L_COL else (M, groups), sdt)
    st = lib().orc_fagq_typed(_ptr(x), _ptr(residual), _ptr(gamma), _ptr(res_out),
                              _ptr(norm_out), _ptr(q), _ptr(scale), M, D, group_size, float(eps),
                              q_format, scale_format, scale_layout, rounding, act_dtype,
                              res_dtype, nthreads)
    if st != 0:
        raise ValueError(f"oracle rejected the arguments (status {st})")
    out = {"residual_out": res_out, "q": q, "scale": scale}
    if with_norm:
        out["norm_out"] = norm_out
    return out


def e4m3fn_to_f64(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.shape, np.float64)
    lib().orc_e4m3fn_to_f64(_ptr(b), _ptr(out), b.size)
    return out


def gemm(a_q: np.ndarray, a_scale: np.ndarray, b_q: np.ndarray, b_scale: np.ndarray,
         a_layout: int = L_COL, nthreads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """The block-scaled GEMM in double.  a_q [M, K], b_q [N, K]: uint8 fp8 bits;
    a_scale: float32 or uint8 (UE8M0), physical [K/128, M] (a_layout L_COL) or
    [M, K/128]; b_scale: float32 or uint8 [ceil(N/128), K/128].  Returns (C,
    bound): C[m, n] and sum_kb |s| sum_k |A B|, both float64 [M, N]."""
    a_q = np.ascontiguousarray(a_q, dtype=np.uint8)
    b_q = np.ascontiguousarray(b_q, dtype=np.uint8)
    a_scale = np.ascontiguousarray(a_scale)
    b_scale = np.ascontiguousarray(b_scale)
    M, K = a_q.shape
    N = b_q.shape[0]
    kb = K // 128
    nb = (N + 127) // 128
    assert b_q.shape[1] == K and K % 128 == 0
    assert a_scale.shape == ((kb, M) if a_layout == L_COL else (M, kb))
    assert b_scale.shape == (nb, kb)
    fmt = lambda s: S_F32 if s.dtype == np.float32 else S_UE8M0
    assert a_scale.dtype in (np.float32, np.uint8) and b_scale.dtype in (np.float32, np.uint8)
    c = np.empty((M, N), np.float64)
    bound = np.empty((M, N), np.float64)
    import os
    st = lib().orc_gemm(_ptr(a_q), _ptr(a_scale), _ptr(b_q), _ptr(b_scale), _ptr(c), _ptr(bound),
                        M, N, K, fmt(a_scale), a_layout, fmt(b_scale),
                        nthreads or min(8, os.cpu_count() or 1))
    if st != 0:
        raise ValueError(f"oracle rejected the arguments (status {st})")
    return c, bound


def fagq_parts(x_parts, residual: np.ndarray, gamma: np.ndarray, eps: float, group_size: int,
               q_format: int = Q_FP8, scale_format: int = S_F32, scale_layout: int = L_ROW,
               rounding: int = R_RNE, nthreads: int = 0) -> dict:
    """The multi-input form: x is the sum of the partial tensors in x_parts
    (uint16 bf16 bits, each [M, D]), added in fp32 in list order before the
    residual.  Returns residual_out, q and scale like fagq()."""
    parts = [np.ascontiguousarray(p, dtype=np.uint16) for p in x_parts]
    residual = np.ascontiguousarray(residual, dtype=np.uint16)
    gamma = np.ascontiguousarray(gamma, dtype=np.uint16)
    M, D = residual.shape
    assert all(p.shape == (M, D) for p in parts) and gamma.shape == (D,)
    groups = D // group_size
    res_out = np.empty((M, D), np.uint16)
    q = np.empty((M, D), np.uint8)
    sdt = np.float32 if scale_format == S_F32 else np.uint8
    scale = np.empty((groups, M) if scale_layout == L_COL else (M, groups), sdt)
    arr = (ctypes.c_void_p * len(parts))(*[p.ctypes.data for p in parts])
    st = lib().orc_fagq_parts(ctypes.cast(arr, ctypes.c_void_p), len(parts), _ptr(residual),
                              _ptr(gamma), _ptr(res_out), None, _ptr(q), _ptr(scale), M, D,
                              group_size, float(eps), q_format, scale_format, scale_layout,
                              rounding, nthreads)
    if st != 0:
        raise ValueError(f"oracle rejected the arguments (status {st})")
    return {"residual_out": res_out, "q": q, "scale": scale}


def dsa_topk(scores: np.ndarray, page_table: np.ndarray, q_pos: np.ndarray, kv_lens: np.ndarray,
             block_size: int, top_k: int, nthreads: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """scores [B, H, Q, NB] float32, or uint16 holding bf16 bits; page_table int32
    [B, NB]; q_pos [B, Q] and kv_lens [B] int32 or int64.  Returns (out_blocks,
    out_pages), int32 [B, H, Q, top_k]."""
    import os
    scores = np.ascontiguousarray(scores)
    assert scores.dtype in (np.float32, np.uint16) and scores.ndim == 4
    B, H, Q, NB = scores.shape
    page_table = np.ascontiguousarray(page_table, dtype=np.int32)
    assert page_table.shape == (B, NB)
    idx64 = q_pos.dtype == np.int64
    idt = np.int64 if idx64 else np.int32
    q_pos = np.ascontiguousarray(q_pos, dtype=idt)
    kv_lens = np.ascontiguousarray(kv_lens, dtype=idt)
    assert q_pos.shape == (B, Q) and kv_lens.shape == (B,)
    ob = np.empty((B, H, Q, top_k), np.int32)
    op = np.empty((B, H, Q, top_k), np.int32)
    st = lib().orc_dsa_topk(_ptr(scores), int(scores.dtype == np.uint16), _ptr(page_table),
                            _ptr(q_pos), _ptr(kv_lens), int(idx64), _ptr(ob), _ptr(op), B, H, Q,
                            NB, block_size, top_k, nthreads or min(8, os.cpu_count() or 1))
    if st != 0:
        raise ValueError(f"oracle rejected the arguments (status {st})")
    return ob, op


def mla_bwd(q: np.ndarray, c: np.ndarray, out: np.ndarray, do: np.ndarray, lse: np.ndarray,
            sm_scale: float, with_bound: bool = True, nthreads: int = 0):
    """The reference's Task 03 operator (oracle/mla_bwd_oracle.c).  q, out, do:
    uint16 bf16 bits [B, H, S, D]; c: uint16 [B, S, D]; lse: float32 [B, H, S].
    Returns (dq float64 [B, H, S, D], dc float64 [B, S, D], dq_bound float64
    [2, B, H, E, D] or None), E = min(16, S): dq_bound[0] = sum_j |dS_ij| |c_jd|,
    dq_bound[1] = the sensitivity of dq to absolute errors in dp - delta
    (oracle/mla_bwd_oracle.c)."""
    import os
    q, c, out, do = (np.ascontiguousarray(a, dtype=np.uint16) for a in (q, c, out, do))
    lse = np.ascontiguousarray(lse, dtype=np.float32)
    B, H, S, D = q.shape
    assert c.shape == (B, S, D) and out.shape == q.shape and do.shape == q.shape
    assert lse.shape == (B, H, S)
    E = min(16, S)
    dq = np.empty((B, H, S, D), np.float64)
    dc = np.empty((B, S, D), np.float64)
    bound = np.empty((2, B, H, E, D), np.float64) if with_bound else None
    st = lib().orc_mla_bwd(_ptr(q), _ptr(c), _ptr(out), _ptr(do), _ptr(lse), _ptr(dq), _ptr(dc),
                           _ptr(bound) if bound is not None else None, B, H, S, D,
                           float(sm_scale), nthreads or min(8, os.cpu_count() or 1))
    if st != 0:
        raise ValueError(f"oracle rejected the arguments (status {st})")
    return dq, dc, bound
