"""The multi-input form (fagq_launch_parts: x is the fp32 sum of partial
tensors) without a GPU: its oracle is pinned against the single-input
oracle, and the C ABI validates its arguments before any device work.

Pins (the form has no counterpart in the reference, so no golden vectors):
* one part is the single-input operator, bit for bit;
* adding a part of negative zeros (x + (-0) = x exactly) changes nothing;
* integer-valued parts whose sum is exact in fp32 and bf16 give the
  single-input result for x = that sum (catches a dropped or repeated part,
  or the residual added before the parts).
"""
import ctypes

import numpy as np
import pytest

import oracle

FORMATS = [(oracle.Q_FP8, oracle.S_F32, oracle.L_COL, oracle.R_RNE),
           (oracle.Q_FP8, oracle.S_UE8M0, oracle.L_COL, oracle.R_RNE),
           (oracle.Q_INT8, oracle.S_F32, oracle.L_ROW, oracle.R_TRUNC)]


def bf16(rng, shape, scale=1.0):
    return oracle.bf16_from_f32((scale * rng.standard_normal(shape)).astype(np.float32))


def same(a, b):
    return all(np.array_equal(a[k], b[k]) for k in ("residual_out", "q", "scale"))


@pytest.mark.parametrize("fmt", FORMATS)
def test_one_part_is_the_operator(fmt):
    rng = np.random.default_rng(1)
    x, r, g = bf16(rng, (9, 1024)), bf16(rng, (9, 1024)), bf16(rng, (1024,), 0.1)
    a = oracle.fagq_parts([x], r, g, 1e-6, 128, *fmt)
    b = oracle.fagq(x, r, g, 1e-6, 128, *fmt)
    assert same(a, b)


@pytest.mark.parametrize("fmt", FORMATS)
def test_negative_zero_parts_change_nothing(fmt):
    rng = np.random.default_rng(2)
    x, r, g = bf16(rng, (7, 2048)), bf16(rng, (7, 2048)), bf16(rng, (2048,), 0.1)
    nz = np.full(x.shape, 0x8000, np.uint16)
    a = oracle.fagq_parts([x, nz, nz, nz], r, g, 1e-6, 128, *fmt)
    b = oracle.fagq(x, r, g, 1e-6, 128, *fmt)
    assert same(a, b)


@pytest.mark.parametrize("nparts", [2, 3, 5, 8])
def test_exact_integer_sums_match_single_input(nparts):
    rng = np.random.default_rng(nparts)
    M, D = 6, 1536
    ints = rng.integers(-12, 13, size=(nparts, M, D)).astype(np.float32)
    parts = [oracle.bf16_from_f32(p) for p in ints]
    total = oracle.bf16_from_f32(ints.sum(0))            # |sum| <= 96: exact in bf16
    r, g = bf16(rng, (M, D), 4.0), bf16(rng, (D,), 0.1)
    a = oracle.fagq_parts(parts, r, g, 1e-6, 128, oracle.Q_FP8, oracle.S_F32, oracle.L_COL)
    b = oracle.fagq(total, r, g, 1e-6, 128, oracle.Q_FP8, oracle.S_F32, oracle.L_COL)
    assert same(a, b)
    # A dropped part is visible.
    c = oracle.fagq_parts(parts[:-1], r, g, 1e-6, 128, oracle.Q_FP8, oracle.S_F32, oracle.L_COL)
    assert not np.array_equal(a["residual_out"], c["residual_out"])


# ----------------------------------------------------------------- C ABI

BASE = 0x10_0000_0000


def fake(i):
    return BASE + i * 0x1_0000_0000


def call(lib, parts=(10, 11), nparts=None, **kw):
    a = dict(residual=fake(1), gamma=fake(2), residual_out=fake(3), q=fake(4), scale=fake(5),
             M=8, D=4096, G=128, eps=1e-6, qf=1, sf=0, layout=1, rounding=0)
    a.update(kw)
    ptrs = [fake(p) if isinstance(p, int) and p < 64 else p for p in parts]
    arr = (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)
    return lib.fagq_launch_parts(ctypes.cast(arr, ctypes.c_void_p),
                                 len(ptrs) if nparts is None else nparts,
                                 ctypes.c_void_p(a["residual"]), ctypes.c_void_p(a["gamma"]),
                                 ctypes.c_void_p(a["residual_out"]), ctypes.c_void_p(a["q"]),
                                 ctypes.c_void_p(a["scale"]), a["M"], a["D"], a["G"], a["eps"],
                                 a["qf"], a["sf"], a["layout"], a["rounding"], None)


def test_parts_validation(lib):
    assert call(lib, M=0) == 0                                     # no-op, no device
    assert call(lib, nparts=0) == 2
    assert call(lib, parts=tuple(range(10, 19))) == 2              # 9 parts
    assert call(lib, parts=(10, None)) == 1
    assert call(lib, parts=(10, BASE + 0xB_0000_0008)) == 4        # misaligned part
    assert call(lib, parts=(10, 4)) == 9                           # part is the code tensor
    assert call(lib, parts=(3, 11)) == 9                           # residual_out is a part
    assert call(lib, D=32768) == 7                                 # above FAGQ_MAX_D_PARTS
    assert call(lib, G=100) == 3
    assert call(lib, residual_out=fake(1), M=0) == 0               # in place on residual
    assert lib.fagq_launch_parts(None, 2, None, None, None, None, None, 8, 4096, 128, 1e-6,
                                 1, 0, 1, 0, None) == 1
