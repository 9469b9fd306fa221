"""Writes the golden fixtures in tests/golden/fagq_golden.npz.

The reference repository holds no golden vectors, fixtures or tests for this
operator, so these fixtures are produced by this repository's C oracle
(oracle/fagq_oracle.c) after it has been pinned against PyTorch's casts,
closed forms and invariants (tests/test_oracle.py).  They freeze the
oracle's outputs, so that a later edit of the oracle that changes any output
bit fails tests/test_golden.py, and they give the GPU library a fixed target.

Each case stores its inputs (bf16 bit patterns) and every output of the
operator.  Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))

import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "fagq_golden.npz"

# (name, M, D, G, q format, scale format, layout, rounding, with norm_out, input scale)
CASES = [
    ("fp8_f32_row_g128", 4, 4096, 128, oracle.Q_FP8, oracle.S_F32, oracle.L_ROW, oracle.R_RNE, False, 1.0),
    ("fp8_f32_col_g128_d7168", 3, 7168, 128, oracle.Q_FP8, oracle.S_F32, oracle.L_COL, oracle.R_RNE, False, 1.0),
    ("fp8_ue8m0_col_g128", 5, 5120, 128, oracle.Q_FP8, oracle.S_UE8M0, oracle.L_COL, oracle.R_RNE, False, 0.5),
    ("int8rne_f32_row_g128", 2, 8192, 128, oracle.Q_INT8, oracle.S_F32, oracle.L_ROW, oracle.R_RNE, False, 1.0),
    ("int8trunc_f32_row_g128_norm", 3, 4096, 128, oracle.Q_INT8, oracle.S_F32, oracle.L_ROW, oracle.R_TRUNC, True, 1.0),
    ("int8trunc_f32_row_g256_norm", 2, 4096, 256, oracle.Q_INT8, oracle.S_F32, oracle.L_ROW, oracle.R_TRUNC, True, 1.0),
    ("fp8_f32_row_g64_ragged", 7, 640, 64, oracle.Q_FP8, oracle.S_F32, oracle.L_ROW, oracle.R_RNE, True, 4.0),
    ("int8rne_ue8m0_row_g64", 1, 1536, 64, oracle.Q_INT8, oracle.S_UE8M0, oracle.L_ROW, oracle.R_RNE, False, 0.01),
]
EPS = 1e-6


def make_case(i: int, M: int, D: int, scale: float):
    rng = np.random.default_rng(1000 + i)
    x = oracle.bf16_from_f32(scale * rng.standard_normal((M, D)).astype(np.float32))
    r = oracle.bf16_from_f32(scale * rng.standard_normal((M, D)).astype(np.float32))
    g = oracle.bf16_from_f32((1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    if M > 1:
        x[1, :] = 0          # an all-zero row
        r[1, :] = 0
        x[1, D // 3] = oracle.bf16_from_f32(np.float32([2.5]))[0]   # ... made one-hot
    return x, r, g


def build() -> dict:
    arrays = {}
    for i, (name, M, D, G, qf, sf, lay, rnd, wn, sc) in enumerate(CASES):
        x, r, g = make_case(i, M, D, sc)
        out = oracle.fagq(x, r, g, EPS, G, qf, sf, lay, rnd, wn)
        meta = np.array([M, D, G, qf, sf, lay, rnd, int(wn)], dtype=np.int64)
        arrays[f"{name}.meta"] = meta
        arrays[f"{name}.x"] = x
        arrays[f"{name}.residual"] = r
        arrays[f"{name}.gamma"] = g
        for k, v in out.items():
            arrays[f"{name}.{k}"] = v
    arrays["eps"] = np.array([EPS], dtype=np.float32)
    return arrays


if __name__ == "__main__":
    arrays = build()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(CASES)} cases)")
