"""ctypes binding of libfagq.so (the C ABI declared in include/fagq.h,
include/fagq_gemm.h, include/fagq_dsa.h, include/fagq_mla.h and
include/fagq_diag.h) and of libfagq_probe.so (include/fagq_probe.h, the
measurement probes, loaded only when asked for).

The library is loaded after ``import torch`` so that its libamdhip64.so.7
dependency resolves to the HIP runtime torch already loaded (same soname);
kernels then run on torch's streams.  There is no fallback: if the library
is missing or does not load, every operator call raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libfagq.so"
PROBE_LIB_PATH = PKG_DIR / "libfagq_probe.so"

# Enums of include/fagq.h and include/fagq_diag.h.
Q_INT8, Q_FP8_E4M3FN = 0, 1
SCALE_F32, SCALE_UE8M0 = 0, 1
LAYOUT_ROW_MAJOR, LAYOUT_COL_MAJOR = 0, 1
ROUND_RNE, ROUND_TRUNC = 0, 1
DT_BF16, DT_F16, DT_F32 = 0, 1, 2
MAX_D = 32768
MAX_PARTS, MAX_D_PARTS = 8, 16384
MODE_INDEPENDENT, MODE_SHARED_GAMMA, MODE_WIDE_SCALES = 0, 1, 2
STREAM_COPY, STREAM_READ, STREAM_WRITE, STREAM_OPMIX = 0, 1, 2, 3

STATUS_NAMES = {
    0: "FAGQ_OK", 1: "FAGQ_E_NULL", 2: "FAGQ_E_SHAPE", 3: "FAGQ_E_GROUP", 4: "FAGQ_E_ALIGN",
    5: "FAGQ_E_FORMAT", 6: "FAGQ_E_EPS", 7: "FAGQ_E_TOO_LARGE", 8: "FAGQ_E_DEVICE",
    9: "FAGQ_E_ALIAS",
}

# Every exported function and its ctypes signature.
_P, _I64, _I, _F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float


class Route(ctypes.Structure):
    _fields_ = [("waves_per_row", ctypes.c_int32), ("steps_per_wave", ctypes.c_int32),
                ("rows_per_block", ctypes.c_int32), ("row_group_mode", ctypes.c_int32),
                ("block_threads", ctypes.c_int32), ("lds_bytes", ctypes.c_int32),
                ("grid_blocks", ctypes.c_int64), ("xcd_remap", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class GemmRoute(ctypes.Structure):
    _fields_ = [("block_m", ctypes.c_int32), ("block_n", ctypes.c_int32),
                ("block_threads", ctypes.c_int32), ("group_m", ctypes.c_int32),
                ("grid_blocks", ctypes.c_int64)]


SIGNATURES = {
    "fagq_launch": ([_P] * 7 + [_I64, _I64, _I64, _F, _I, _I, _I, _I, _P], _I),
    "fagq_launch_typed": ([_P] * 7 + [_I64, _I64, _I64, _F, _I, _I, _I, _I, _I, _I, _P], _I),
    "fagq_launch_parts": ([_P, _I] + [_P] * 5 + [_I64, _I64, _I64, _F, _I, _I, _I, _I, _P], _I),
    "fagq_launch_mapped": ([_P] * 7 + [_I64, _I64, _I64, _F] + [_I] * 9 + [_P], _I),
    "fagq_query_route": ([_I64, _I64, _I64, _I, _I, ctypes.POINTER(Route)], _I),
    "fagq_query_route_typed": ([_I64, _I64, _I64, _I, _I, _I, _I, ctypes.POINTER(Route)], _I),
    "fagq_query_route_parts": ([_I64, _I64, _I64, _I, _I, _I, ctypes.POINTER(Route)], _I),
    "fagq_status_string": ([_I], ctypes.c_char_p),
    "fagq_version": ([], _I),
    "fagq_diag_encode": ([_P, _P, _I64, _I, _I, _I, _P], _I),
    "fagq_diag_scale_offsets": ([_I64, _I64, _I64, _I, _I, _I, _I64, _P, _I64], _I),
    "fagq_dsa_topk_launch": ([_P, _I, _P, _P, _P, _I, _P, _P] + [_I64] * 6 + [_P], _I),
    "fagq_gemm_launch": ([_P] * 5 + [_I64, _I64, _I64, _I, _I, _I, _P], _I),
    "fagq_gemm_launch_mapped": ([_P] * 5 + [_I64, _I64, _I64, _I, _I, _I, _I, _P], _I),
    "fagq_gemm_query_route": ([_I64, _I64, _I64, ctypes.POINTER(GemmRoute)], _I),
    "fagq_mla_bwd_workspace_bytes": ([_I64, _I64, _I64], _I64),
    "fagq_mla_bwd_launch": ([_P] * 8 + [_I64] * 5 + [_F, _I, _I, _P], _I),
    "fagq_mla_bwd_launch_noalloc": ([_P] * 7 + [_I64] * 4 + [_F, _I, _I, _P], _I),
}


# libfagq_probe.so (include/fagq_probe.h).
PROBE_SIGNATURES = {
    "fagq_diag_copy": ([_P, _P, _I64, _P], _I),
    "fagq_diag_stream": ([_P, _P, _I64, _I, _P], _I),
    "fagq_diag_mfma_peak": ([_P, _I64, _I, _P], _I),
    "fagq_diag_mfma_rate": ([_P, _I64, _I, _I, _P], _I),
    "fagq_diag_lds_read": ([_P, _I64, _I, _I, _P], _I),
}


class FagqError(RuntimeError):
    """A non-zero status from the library."""

    def __init__(self, status: int, what: str = "fagq_launch"):
        self.status = status
        name = STATUS_NAMES.get(status, "HIP error" if status < 0 else "unknown")
        super().__init__(f"{what} failed: status {status} ({name}): {describe(status)}")


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_probe: ctypes.CDLL | None = None


def _open(p: Path, signatures: dict) -> ctypes.CDLL:
    if not p.exists():
        raise ImportError(
            f"{p} is missing: build the HIP libraries first "
            "(python __graft_entry__.py build, or build.build())")
    lib = ctypes.CDLL(str(p))
    for name, (args, res) in signatures.items():
        fn = getattr(lib, name)   # AttributeError if an export is missing
        fn.argtypes = args
        fn.restype = res
    return lib


def load(path: str | Path | None = None) -> ctypes.CDLL:
    """Loads libfagq.so once; raises if it is absent or incomplete."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        lib = _open(Path(path) if path is not None else LIB_PATH, SIGNATURES)
        if path is None:
            _lib = lib
        return lib


def load_probe(path: str | Path | None = None) -> ctypes.CDLL:
    """Loads libfagq_probe.so (the measurement probes) once; raises if it is
    absent or incomplete."""
    global _probe
    if _probe is not None and path is None:
        return _probe
    with _lock:
        if _probe is not None and path is None:
            return _probe
        lib = _open(Path(path) if path is not None else PROBE_LIB_PATH, PROBE_SIGNATURES)
        if path is None:
            _probe = lib
        return lib


_fast = None          # the bound _fagq_py.launch, once looked up
_fast_tried = False


def fast_launch():
    """launch() of the CPython binding (csrc/fagq_py.cpp), bound to this
    process's libfagq.so, or None when that module is not built or does not
    import (the ctypes path then serves every call; both reach fagq_launch)."""
    global _fast, _fast_tried
    if _fast_tried:
        return _fast
    lib = load()          # takes _lock itself (not reentrant): before the block below
    with _lock:
        if not _fast_tried:
            try:
                from . import _fagq_py
                _fagq_py.bind(ctypes.cast(lib.fagq_launch, ctypes.c_void_p).value,
                              ctypes.cast(lib.fagq_launch_typed, ctypes.c_void_p).value)
                _fast = _fagq_py.launch
            except ImportError:
                _fast = None
            _fast_tried = True
    return _fast


FAST_ARG_ERROR = 1000   # _fagq_py.ARG_ERROR: a tensor argument was rejected by the binding


def describe(status: int) -> str:
    try:
        return load().fagq_status_string(status).decode()
    except Exception:  # pragma: no cover - only when the library cannot load
        return STATUS_NAMES.get(status, "unknown")


def check(status: int, what: str = "fagq_launch") -> None:
    if status != 0:
        raise FagqError(status, what)


def query_route(M: int, D: int, group_size: int, scale_format: int = SCALE_F32,
                scale_layout: int = LAYOUT_ROW_MAJOR, act_dtype: int | None = None,
                res_dtype: int | None = None) -> dict:
    """The route of fagq_launch, or of fagq_launch_typed when element types are given."""
    r = Route()
    if act_dtype is None and res_dtype is None:
        check(load().fagq_query_route(M, D, group_size, scale_format, scale_layout,
                                      ctypes.byref(r)), "fagq_query_route")
    else:
        act = DT_BF16 if act_dtype is None else act_dtype
        res = act if res_dtype is None else res_dtype
        check(load().fagq_query_route_typed(M, D, group_size, scale_format, scale_layout, act, res,
                                            ctypes.byref(r)), "fagq_query_route_typed")
    return {f: getattr(r, f) for f, _ in Route._fields_ if f != "reserved"}


def query_route_parts(M: int, D: int, group_size: int, nparts: int,
                      scale_format: int = SCALE_F32, scale_layout: int = LAYOUT_ROW_MAJOR) -> dict:
    """The route of fagq_launch_parts for nparts partials."""
    r = Route()
    check(load().fagq_query_route_parts(M, D, group_size, nparts, scale_format, scale_layout,
                                        ctypes.byref(r)), "fagq_query_route_parts")
    return {f: getattr(r, f) for f, _ in Route._fields_ if f != "reserved"}
