"""Per-lane scale addressing of the operator's kernels, checked on the host.

fagq_diag_scale_offsets evaluates, with the same functions the kernels use
(scale_span, scale_lane_offset in csrc/fagq_kernels.hpp), which scale element
every lane of every wave stores for one row, or -1 when the buffer descriptor
drops the store.  Expected: a lane holding columns c..c+7 of the row stores
the scale of group c // G at [row, g] (row-major) or [g, row] (column-major)
when c < D, and nothing when c >= D.  The edge shapes put the 32-bit offsets
of lanes past the row end at or beyond 2^32, where a wrapped offset would land
inside the descriptor and overwrite a real scale."""
import ctypes
import math

import numpy as np
import pytest


def offsets(lib, M, D, G, sf, layout, wpr, row):
    steps = math.ceil(D / 512)
    ns = math.ceil(steps / wpr)
    out = np.full(wpr * ns * 64, -7, dtype=np.int64)
    st = lib.fagq_diag_scale_offsets(M, D, G, sf, layout, wpr, row,
                                     out.ctypes.data_as(ctypes.c_void_p), out.size)
    return st, out.reshape(wpr, ns, 64), ns


def expected(M, D, G, layout, wpr, ns, row):
    groups = D // G
    e = np.full((wpr, ns, 64), -1, dtype=np.int64)
    for p in range(wpr):
        for k in range(ns):
            for lane in range(64):
                c = (p * ns + k) * 512 + lane * 8
                if c < D:
                    g = c // G
                    e[p, k, lane] = g * M + row if layout == 1 else row * groups + g
    return e


CASES = [
    # (M, D, G, scale format, layout, waves per row)
    (16384, 7168, 128, 0, 1, 7), (16384, 7168, 128, 0, 1, 4), (16384, 7168, 128, 0, 1, 14),
    (16384, 7168, 128, 0, 0, 7), (8192, 5120, 128, 1, 1, 5), (8192, 5120, 128, 1, 1, 3),
    (4096, 4096, 128, 0, 0, 4), (1, 8192, 128, 0, 0, 16), (19, 4160, 64, 0, 1, 3),
    (5, 768, 256, 1, 0, 2),
    # Lanes past a short row: group index up to 7 (G = 64) or 3 (G = 128) with
    # g * M * sb reaching 2^32 (fp32: M = 2^28 rows; ue8m0: M = 2^30 rows).
    (1 << 28, 64, 64, 0, 1, 1), ((1 << 28) - 3, 64, 64, 0, 1, 1), (1 << 30, 64, 64, 1, 1, 1),
    (1 << 30, 128, 128, 1, 1, 1), ((1 << 30) + 5, 128, 128, 1, 1, 1),
    # Within the column-major limit (M * groups * sb < 2^32 - 16) a relative group
    # index can pass 2^32 / (M * sb) only in a row shorter than one wave's
    # columns, as above; longer rows at large M for completeness.
    (1 << 26, 192, 64, 0, 1, 1), (3 << 28, 64, 64, 1, 1, 1), ((1 << 24) + 7, 6208, 64, 1, 1, 4),
]


@pytest.mark.parametrize("M,D,G,sf,layout,wpr", CASES)
def test_every_lane_stores_its_group_or_nothing(lib, M, D, G, sf, layout, wpr):
    sb = 4 if sf == 0 else 1
    if layout == 1 and M * (D // G) * sb > (1 << 32) - 17:
        pytest.skip("beyond the column-major limit (checked below)")
    for row in sorted({0, 1 % M, M // 2, M - 1}):
        st, got, ns = offsets(lib, M, D, G, sf, layout, wpr, row)
        assert st == 0, st
        want = expected(M, D, G, layout, wpr, ns, row)
        bad = np.argwhere(got != want)
        assert bad.size == 0, (row, bad[:4], got[tuple(bad[0])], want[tuple(bad[0])])


def test_every_group_of_a_row_is_stored():
    """The expectation itself covers each group of the row with exactly G / 8 lanes."""
    for M, D, G, sf, layout, wpr in CASES[:10]:
        ns = math.ceil(math.ceil(D / 512) / wpr)
        e = expected(M, D, G, layout, wpr, ns, 3 % M)
        vals, counts = np.unique(e[e >= 0], return_counts=True)
        assert len(vals) == D // G and (counts == G // 8).all()


def test_column_major_limit(lib):
    """Column-major scale spans must stay below 2^32 - 16 bytes, so that the
    out-of-range offset 0xffffffff can never land."""
    out = np.zeros(64, dtype=np.int64)
    p = out.ctypes.data_as(ctypes.c_void_p)
    M = ((1 << 32) - 17) // 4          # groups = 1, fp32: M * 4 <= 2^32 - 17
    assert lib.fagq_diag_scale_offsets(M, 64, 64, 0, 1, 1, 0, p, 64) == 0
    assert lib.fagq_diag_scale_offsets(M + 1, 64, 64, 0, 1, 1, 0, p, 64) == 7
    assert lib.fagq_diag_scale_offsets((1 << 25), 7168, 128, 0, 1, 7, 0, p, 64 * 14) == 7


def test_scale_offsets_validation(lib):
    out = np.zeros(64, dtype=np.int64)
    p = out.ctypes.data_as(ctypes.c_void_p)
    assert lib.fagq_diag_scale_offsets(8, 4096, 128, 0, 0, 8, 0, None, 64) == 1
    assert lib.fagq_diag_scale_offsets(8, 4096, 100, 0, 0, 8, 0, p, 64 * 8) == 3
    assert lib.fagq_diag_scale_offsets(8, 4096, 128, 0, 0, 8, 8, p, 64 * 8) == 2   # row >= M
    assert lib.fagq_diag_scale_offsets(8, 4096, 128, 0, 0, 8, 0, p, 64 * 8 - 1) == 2  # cap
    assert lib.fagq_diag_scale_offsets(8, 4096, 128, 0, 0, 1, 0, p, 64 * 8) == 5   # 8 steps/wave
    assert lib.fagq_diag_scale_offsets(8, 4096, 128, 2, 0, 8, 0, p, 64 * 8) == 5
