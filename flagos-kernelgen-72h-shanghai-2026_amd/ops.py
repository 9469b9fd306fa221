"""The operator's Python interface, mirroring the reference's.

``fused_add_rmsnorm_group_quant`` keeps the reference's signature and
semantics (src/task01_fused_add_rmsnorm_group_quant.py:1731-1741, returns at
:1764/:1790/:1817/:1840/:1851): the caller allocates every output, the call
is asynchronous on torch's current stream, and the same four objects are
returned.  The output formats are read from the destination tensors:

* ``x_q`` int8 -> int8 codes, rounded toward zero like the reference's
  float->int cast (:112-116, :1100-1104) unless ``rounding="rne"``;
  ``x_q`` float8_e4m3fn -> OCP fp8 codes, round to nearest even.
* ``x_scale`` float32 -> fp32 scales; uint8 -> UE8M0 biased exponents.
* ``x_scale`` contiguous [M, D/G] -> row-major (the reference's layout,
  :121); a [M, D/G] view with strides (1, M), e.g.
  ``torch.empty(D // G, M).t()``, -> column-major.
* ``norm_out`` may be None: the 3-output form, which skips 2 bytes/element.
* Element types, as the reference's kernels convert them (loads to fp32,
  stores rounded to the destination's type, task01.py:88-94, :91, :118):
  ``x``, ``gamma`` and ``norm_out`` share one type and ``residual``,
  ``residual_out`` another, with (x, residual) in (bf16, bf16), (fp16, fp16),
  (bf16, fp32), (fp16, fp32) or (fp32, fp32).  bf16 runs through
  ``fagq_launch``, the others through ``fagq_launch_typed``.

The reference validates nothing; here shapes, dtypes, devices and layouts
are checked in Python (TypeError / ValueError) and everything else by the
library (FagqError with its status code).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_BF16 = torch.bfloat16
_F16 = torch.float16
_FP8 = torch.float8_e4m3fn
_DT_CODE = {torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16,
            torch.float32: _lib.DT_F32}
# (x dtype, residual dtype) pairs the library takes.
_PAIRS = {(_lib.DT_BF16, _lib.DT_BF16), (_lib.DT_F16, _lib.DT_F16), (_lib.DT_BF16, _lib.DT_F32),
          (_lib.DT_F16, _lib.DT_F32), (_lib.DT_F32, _lib.DT_F32)}


def _q_format(x_q: torch.Tensor) -> int:
    if x_q.dtype is _FP8:
        return _lib.Q_FP8_E4M3FN
    if x_q.dtype is torch.int8:
        return _lib.Q_INT8
    raise TypeError(f"x_q must be int8 or float8_e4m3fn, got {x_q.dtype}")


def _scale_format(x_scale: torch.Tensor) -> int:
    if x_scale.dtype is torch.float32:
        return _lib.SCALE_F32
    if x_scale.dtype is torch.uint8:
        return _lib.SCALE_UE8M0
    raise TypeError(f"x_scale must be float32 or uint8 (ue8m0), got {x_scale.dtype}")


def _scale_layout(x_scale: torch.Tensor, M: int, groups: int) -> int:
    if x_scale.shape != (M, groups):
        raise ValueError(f"x_scale must have shape ({M}, {groups}), got {tuple(x_scale.shape)}")
    if x_scale.is_contiguous():
        return _lib.LAYOUT_ROW_MAJOR
    if x_scale.stride() == (1, M):
        return _lib.LAYOUT_COL_MAJOR
    raise ValueError(f"x_scale must be row-major [M, D/G] or column-major (strides (1, M)); "
                     f"got strides {x_scale.stride()}")


def _rounding(rounding: str | None, q_format: int) -> int:
    if q_format == _lib.Q_FP8_E4M3FN:
        if rounding not in (None, "rne"):
            raise ValueError("fp8 codes are always rounded to nearest even")
        return _lib.ROUND_RNE
    if rounding in (None, "trunc"):
        return _lib.ROUND_TRUNC
    if rounding == "rne":
        return _lib.ROUND_RNE
    raise ValueError(f"rounding must be 'rne' or 'trunc', got {rounding!r}")


def _check_rows(name: str, t: torch.Tensor, shape: tuple, device: torch.device,
                dtype: torch.dtype = _BF16) -> None:
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {str(dtype).replace('torch.', '')}, got {t.dtype}")
    if tuple(t.shape) != shape:
        raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


# Per-call host work is what bounds decode-sized calls (the kernel takes about
# 3 us, the HIP launch about 3.3 us of host time).  The hot path hands the
# tensors to the CPython binding (csrc/fagq_py.cpp), which checks them on their
# C++ metadata and calls fagq_launch; the current device and stream come from
# torch's raw accessors (no torch.device / Stream objects).  Without the
# binding, or when the tensors are not on the current device, the Python path
# below checks every tensor inline in one pass and calls fagq_launch through
# ctypes (entering a device guard only when needed), falling back to the
# detailed checks only to word an error.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_raw_device = getattr(torch._C, "_cuda_getDevice", None)
_INT8 = torch.int8
_F32 = torch.float32
_U8 = torch.uint8
_Q_CODE = {_FP8: _lib.Q_FP8_E4M3FN, _INT8: _lib.Q_INT8}
_S_CODE = {_F32: _lib.SCALE_F32, _U8: _lib.SCALE_UE8M0}
_ROUNDING_CODE = {None: -1, "rne": 0, "trunc": 1}   # the binding's rounding argument


def _current_stream(dev: int) -> int:
    if _raw_stream is not None:
        return _raw_stream(dev)
    return torch.cuda.current_stream(dev).cuda_stream


def _is_current(dev: int) -> bool:
    return (_raw_device() if _raw_device is not None else torch.cuda.current_device()) == dev


def _rows_ok(t, shape, dev: int, dtype=_BF16) -> bool:
    return (t.dtype is dtype and t.shape == shape and t.get_device() == dev
            and t.is_contiguous())


def _launch(fn, dev: int, args) -> int:
    if _is_current(dev):
        return fn(*args, _current_stream(dev))
    with torch.cuda.device(dev):
        return fn(*args, _current_stream(dev))


def _explain(x, residual, gamma, residual_out, norm_out, x_q, x_scale, group_size, rounding):
    """Raises the detailed error for arguments the fast checks rejected."""
    M, D = (int(v) for v in x.shape)
    device = x.device
    if x.dtype not in _DT_CODE:
        raise TypeError(f"x must be bfloat16, float16 or float32, got {x.dtype}")
    if residual.dtype not in _DT_CODE:
        raise TypeError(f"residual must be bfloat16, float16 or float32, got {residual.dtype}")
    if (_DT_CODE[x.dtype], _DT_CODE[residual.dtype]) not in _PAIRS:
        raise TypeError(f"unsupported (x, residual) dtypes ({x.dtype}, {residual.dtype}): "
                        "residual must have x's dtype or be float32")
    _check_rows("x", x, (M, D), device, x.dtype)
    _check_rows("residual", residual, (M, D), device, residual.dtype)
    _check_rows("gamma", gamma, (D,), device, x.dtype)
    _check_rows("residual_out", residual_out, (M, D), device, residual.dtype)
    if norm_out is not None:
        _check_rows("norm_out", norm_out, (M, D), device, x.dtype)
    if group_size <= 0 or D % group_size != 0:
        raise ValueError(f"group_size {group_size} must divide D = {D}")
    qf = _q_format(x_q)
    if x_q.device != device or tuple(x_q.shape) != (M, D) or not x_q.is_contiguous():
        raise ValueError(f"x_q must be a contiguous ({M}, {D}) tensor on {device}")
    if x_scale.device != device:
        raise ValueError(f"x_scale is on {x_scale.device}, expected {device}")
    _scale_format(x_scale)
    _scale_layout(x_scale, M, D // group_size)
    _rounding(rounding, qf)
    raise ValueError("invalid arguments")    # not reached: one of the checks above raises


def fused_add_rmsnorm_group_quant(
    x: torch.Tensor,
    residual: torch.Tensor,
    gamma: torch.Tensor,
    residual_out: torch.Tensor,
    norm_out: torch.Tensor | None,
    x_q: torch.Tensor,
    x_scale: torch.Tensor,
    eps: float,
    group_size: int,
    *,
    rounding: str | None = None,
):
    """residual_out = x + residual; x_q, x_scale = group-quant(RMSNorm(x + residual) * gamma).

    Drop-in for the reference's operator of the same name and signature; see
    the module docstring for how the formats are chosen.  Returns
    ``(residual_out, norm_out, x_q, x_scale)``.
    """
    fast = _lib._fast if _lib._fast_tried else _lib.fast_launch()
    if fast is not None and _raw_device is not None and _raw_stream is not None \
            and type(eps) is float:
        dev = x.get_device()
        if dev >= 0 and _raw_device() == dev:
            st = fast(x, residual, gamma, residual_out, norm_out, x_q, x_scale, eps, group_size,
                      _ROUNDING_CODE.get(rounding, -2) if isinstance(rounding, (str, type(None)))
                      else -2, _raw_stream(dev))
            if st == 0:
                return residual_out, norm_out, x_q, x_scale
            if st != _lib.FAST_ARG_ERROR:
                _lib.check(st)
            # A rejected argument: the checks below raise the detailed error.
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [M, D], got shape {tuple(x.shape)}")
    dev = x.get_device()
    if dev < 0:
        raise ValueError("x must be a GPU (HIP) tensor; this operator has no CPU path")
    shape = x.shape
    M, D = shape
    G = int(group_size)
    qf = _Q_CODE.get(x_q.dtype)
    sf = _S_CODE.get(x_scale.dtype)
    ss = x_scale.shape
    xt, rt = x.dtype, residual.dtype
    act, res = _DT_CODE.get(xt), _DT_CODE.get(rt)
    if not ((act, res) in _PAIRS and x.is_contiguous()
            and residual.shape == shape
            and residual.get_device() == dev and residual.is_contiguous()
            and residual_out.dtype is rt and residual_out.shape == shape
            and residual_out.get_device() == dev and residual_out.is_contiguous()
            and (norm_out is None or _rows_ok(norm_out, shape, dev, xt))
            and gamma.dtype is xt and gamma.shape == (D,) and gamma.get_device() == dev
            and gamma.is_contiguous()
            and G > 0 and D % G == 0
            and qf is not None and x_q.shape == shape and x_q.get_device() == dev
            and x_q.is_contiguous()
            and sf is not None and x_scale.get_device() == dev and len(ss) == 2
            and ss[0] == M and ss[1] == D // G):
        _explain(x, residual, gamma, residual_out, norm_out, x_q, x_scale, G, rounding)
    if x_scale.is_contiguous():
        layout = _lib.LAYOUT_ROW_MAJOR
    else:
        layout = _scale_layout(x_scale, M, D // G)
    if rounding is None:
        rnd = _lib.ROUND_RNE if qf == _lib.Q_FP8_E4M3FN else _lib.ROUND_TRUNC
    else:
        rnd = _rounding(rounding, qf)
    if M == 0:
        return residual_out, norm_out, x_q, x_scale
    L = _lib._lib or _lib.load()
    args = (x.data_ptr(), residual.data_ptr(), gamma.data_ptr(), residual_out.data_ptr(),
            None if norm_out is None else norm_out.data_ptr(), x_q.data_ptr(), x_scale.data_ptr(),
            M, D, G, float(eps), qf, sf, layout, rnd)
    if act == _lib.DT_BF16 and res == _lib.DT_BF16:
        fn = L.fagq_launch
    else:
        fn = L.fagq_launch_typed
        args = args + (act, res)
    if _raw_device is not None and _raw_stream is not None and _raw_device() == dev:
        st = fn(*args, _raw_stream(dev))
    else:
        st = _launch(fn, dev, args)
    if st:
        _lib.check(st)
    return residual_out, norm_out, x_q, x_scale


def empty_scales(M: int, groups: int, *, ue8m0: bool = False, col_major: bool = False,
                 device=None) -> torch.Tensor:
    """A [M, groups] scale tensor in the requested format and layout."""
    dt = torch.uint8 if ue8m0 else torch.float32
    if col_major:
        return torch.empty(groups, M, dtype=dt, device=device).t()
    return torch.empty(M, groups, dtype=dt, device=device)


def fused_add_rmsnorm_group_quant_fn(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    group_size: int = 128,
    out_dtype: torch.dtype = _FP8,
    *,
    scale_col_major: bool = False,
    scale_ue8m0: bool = False,
    rounding: str = "rne",
    inplace_residual: bool = False,
):
    """Functional 3-output form: returns ``(residual_out, q, scale)``.

    ``residual_out`` is ``residual`` itself when ``inplace_residual`` (the
    "updated residual" of a transformer block), else a new tensor.  ``scale``
    is a [M, D/G] tensor, column-major when ``scale_col_major``, holding
    UE8M0 bytes when ``scale_ue8m0``.  int8 codes default to round-half-even
    here (the reference-signature function defaults to truncation).
    """
    M, D = (int(s) for s in x.shape)
    residual_out = residual if inplace_residual else torch.empty_like(residual)
    q = torch.empty((M, D), dtype=out_dtype, device=x.device)
    scale = empty_scales(M, D // group_size, ue8m0=scale_ue8m0, col_major=scale_col_major,
                         device=x.device)
    fused_add_rmsnorm_group_quant(x, residual, weight, residual_out, None, q, scale, eps,
                                  group_size, rounding=None if out_dtype == _FP8 else rounding)
    return residual_out, q, scale


def fused_reduce_add_rmsnorm_group_quant(
    x_parts,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
    group_size: int = 128,
    out_dtype: torch.dtype = _FP8,
    *,
    scale_col_major: bool = False,
    scale_ue8m0: bool = False,
    rounding: str = "rne",
    inplace_residual: bool = False,
):
    """Multi-input form (the epilogue of a tensor-parallel reduction): x is the
    sum of the partial tensors in ``x_parts`` (1 to 8 bf16 [M, D] tensors, one per
    rank), added in fp32 in list order before the residual and never rounded to
    bf16.  Returns ``(residual_out, q, scale)`` like the functional form; with one
    part the outputs equal it bit for bit.  C ABI: ``fagq_launch_parts``.

    No counterpart in the reference (its operator takes one x,
    src/task01_fused_add_rmsnorm_group_quant.py:1731-1741).
    """
    parts = list(x_parts)
    if not 1 <= len(parts) <= 8:
        raise ValueError(f"x_parts must hold 1 to 8 tensors, got {len(parts)}")
    x0 = parts[0]
    if x0.dim() != 2:
        raise ValueError(f"x_parts[0] must be 2-D [M, D], got shape {tuple(x0.shape)}")
    if not x0.is_cuda:
        raise ValueError("x_parts must be GPU (HIP) tensors; this operator has no CPU path")
    M, D = (int(s) for s in x0.shape)
    device = x0.device
    for i, t in enumerate(parts):
        _check_rows(f"x_parts[{i}]", t, (M, D), device)
    _check_rows("residual", residual, (M, D), device)
    _check_rows("weight", weight, (D,), device)
    group_size = int(group_size)
    if group_size <= 0 or D % group_size != 0:
        raise ValueError(f"group_size {group_size} must divide D = {D}")
    residual_out = residual if inplace_residual else torch.empty_like(residual)
    q = torch.empty((M, D), dtype=out_dtype, device=device)
    scale = empty_scales(M, D // group_size, ue8m0=scale_ue8m0, col_major=scale_col_major,
                         device=device)
    qf = _q_format(q)
    sf = _scale_format(scale)
    layout = _scale_layout(scale, M, D // group_size)
    rnd = _rounding(None if out_dtype == _FP8 else rounding, qf)
    if M == 0:
        return residual_out, q, scale
    arr = (ctypes.c_void_p * len(parts))(*[t.data_ptr() for t in parts])
    st = _launch(_lib.load().fagq_launch_parts, x0.get_device(),
                 (ctypes.cast(arr, ctypes.c_void_p), len(parts), residual.data_ptr(),
                  weight.data_ptr(), residual_out.data_ptr(), q.data_ptr(), scale.data_ptr(), M, D,
                  group_size, float(eps), qf, sf, layout, rnd))
    _lib.check(st, "fagq_launch_parts")
    return residual_out, q, scale


def route_for(M: int, D: int, group_size: int = 128, *, scale_ue8m0: bool = False,
              scale_col_major: bool = False, x_dtype: torch.dtype = torch.bfloat16,
              residual_dtype: torch.dtype | None = None) -> dict:
    """The launch mapping the library chooses for a shape, scale format and
    element types (x / gamma / norm_out, residual / residual_out; the
    residual stream defaults to x's type)."""
    rt = x_dtype if residual_dtype is None else residual_dtype
    if x_dtype not in _DT_CODE or rt not in _DT_CODE:
        raise TypeError(f"unsupported (x, residual) dtypes ({x_dtype}, {rt})")
    sf = _lib.SCALE_UE8M0 if scale_ue8m0 else _lib.SCALE_F32
    layout = _lib.LAYOUT_COL_MAJOR if scale_col_major else _lib.LAYOUT_ROW_MAJOR
    if x_dtype is torch.bfloat16 and rt is torch.bfloat16:
        return _lib.query_route(M, D, group_size, sf, layout)
    return _lib.query_route(M, D, group_size, sf, layout, _DT_CODE[x_dtype], _DT_CODE[rt])
